// int32 convolution on quantized float codes (the reference's launch_fprop_nhwc_qi32<Tin>,
// /root/reference/src/conv_types.h:308-323 -> cuda_kernels.cu:1336-1392) on the int8 row-band
// structure: each float code is read from HBM once per band, staged in LDS as one int8 value,
// and the MFMA loop is that of the int8 band kernel (v_mfma_i32_16x16x64_i8, filter in
// registers).  The result is the reference's CPU definition (cpu_ref.cpp:36-72):
//   y[n,ho,wo,g*Kg+k] = sum over in-bounds taps (int32(x) - zx[n]) * (int32(w) - zw)
// with int32 wrap-around and int32() truncating toward zero.
//
// Offset codes.  With a fixed offset o (128 for LinQuantU8 codes, 0 for LinQuantS5) the staged
// values are x' = int32(x) - o and w' = int32(w) - o, which are int8 for codes of the
// parameter type's range.  A padded tap is staged as x' = zx - o, so that x' + (o - zx) = 0:
// it contributes nothing, which is the reference's skip.  With dx = o - zx and dw = o - zw,
// over all R*S*(C/groups) = Kdim terms of the window
//   y = sum x'w' + dw * W(p) + dx * T(k) + Kdim * dx * dw            (mod 2^32)
// where W(p) is the sum of the pixel's staged window and T(k) the sum of channel k's staged
// filter row.  The accumulators start at dx * T(k) + Kdim * dx * dw (one image and one
// filter per workgroup); the epilogue adds dw * W(p), W(p) being the sum of KB per-pixel
// channel sums staged beside the rows.
//
// Range.  A code whose offset value lies outside [-128, 127] (any float is allowed: wide,
// negative or fractional codes) marks its wave; after staging, a workgroup with a marked wave
// computes its outputs by direct VALU arithmetic on the float codes instead, exact as well.
//
// Work decomposition, input-row layout, segment walk and skew are those of the int8 band
// kernel: a workgroup of 8 waves owns BH output rows of one image and NT 64-channel tiles of
// one group;  with blocked filters (the reference's launch_block_fprop_nhwc_qi32, output pixel
// (ho, wo) taking filter block (ho / block_ho, wo / block_wo)) its rows and columns lie inside
// one block (a band never crosses a block row; its columns are the block's block_wo) and it
// loads that block's filter tiles; each wave keeps its tile's filter in registers (KB = R*S*(C/groups)/64 K-blocks);
// 16-pixel segments run one per phase.  Output channels are not permuted: MFMA row block j
// holds channels 16j .. 16j + 15, so the 4 lanes of a pixel store 64 contiguous bytes of int32.
//
// Filter prepass.  A small kernel converts the filter once per call to offset int8 in MFMA
// fragment order (and a range flag per 64-channel tile and K-block) into a caller workspace;
// each band workgroup then loads its tiles by DMA (1 KB per buffer_load ... lds), as the int8
// band kernel loads its filter.  Converting the float filter in every workgroup instead read
// 147 KB per CU from L2 on C2 and took ~9 us of its 24.
//
// Staging.  Input codes come in 16-byte buffer loads of 4 codes into registers (the values
// must be converted), 1 KB contiguous per wave instruction when C/groups == 64, 4 in flight
// per lane; each lane writes its 4 converted values as one LDS word.  The compiler's own waits
// order them (buffer loads are counted by vmcnt alone).  After a barrier the filter row sums and
// the per-column channel sums are read back from LDS (v_dot4 against ones) and the filter is
// copied into registers.

#include "qconv_device.h"

#include <algorithm>
#include <atomic>

namespace miq {
namespace {

constexpr int kQbWaves = 8;
constexpr int kQbMaxKB = 9;
constexpr int kQbLds = 160 * 1024;
// LDS of one 64-channel tile's filter in 16-byte slots: KB K-blocks x 4 fragments of 1 KB
__host__ __device__ constexpr int qb_tile_slots(int KB) { return 256 * KB; }

struct Qi32BandArgs {
  const float* x;
  const float* w;
  int32_t* y;
  const unsigned char* in_qp;
  const unsigned char* f_qp;
  const int8_t* wfrag;  // the filter prepass's int8 fragments; its range flags follow at byte flags_off
  int flags_off;
  int H, W, C, K, Ho, Wo;
  int ph, pw, sh, dh, dw, R, S;
  int Cg, Kg;
  int BH, bands_per_img, NT, kt_per_group, nblocks;
  int NQ, NPB, SEGR;
  int dS, d_rb, c_rb, d_out, c_out;  // segment walk, as in the int8 band kernel
  int ni;                            // input units per workgroup = HR * NQ * NPB
  int halo_lds;                      // LDS byte offset of the rows (the filter is at 0); column sums, filter sums, wave marks follow
  int tap[kQbMaxKB];                 // K-block b: halo slot offset of (filter row, quad) << 8 | column shift
  int ntiles;
  int Wb, bho, Bx, bpb;              // columns per workgroup (a block's), rows per block, column blocks, bands per block
  FastDivM fd_ntiles, fd_bpi, fd_ktpg, fd_rowi, fd_npb, fd_bpb, fd_bx;
};

static_assert(sizeof(Qi32BandArgs) <= 320, "kernel arguments fit one batch of s_load instructions");

// Per-sample zero point from the raw parameter struct: uint8 at offset 0 of a 12-byte struct
// (LinQuantU8), int8 at offset 0 of an 8-byte struct (LinQuantS5).  A buffer load (counted by
// vmcnt alone): a flat load would make the compiler wait for every load issued before its use.
template <QpKind Q>
__device__ __forceinline__ int qb_zero_point(const unsigned char* qp, int i) {
  constexpr int kStride = Q == kQpU8 ? 12 : 8;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(qp + static_cast<size_t>(i) * kStride, 4);
  const int word = __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0);
  if constexpr (Q == kQpU8) {
    return word & 0xff;
  } else {
    return static_cast<int>(static_cast<signed char>(word & 0xff));
  }
}

// 4 codes -> 4 offset int8 values in one word; `bad` is set when one of them lies outside
// int8.  Invalid (padded) positions take `pad`.
__device__ __forceinline__ unsigned qb_pack4(const v4f& v, bool valid, unsigned off, unsigned pad, bool& bad) {
  unsigned word = 0;
  bool b = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const unsigned u = valid ? static_cast<unsigned>(static_cast<int32_t>(v[e])) - off : pad;
    b |= (u + 128u) > 255u;
    word |= (u & 0xffu) << (8 * e);
  }
  bad = bad || b;
  return word;
}

// Sum of the 16 signed bytes of a 16-byte word.
__device__ __forceinline__ int qb_bytesum(const v4i& v) {
  int s = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) s = __builtin_amdgcn_sdot4(v[d], 0x01010101, s, false);
  return s;
}

__device__ __forceinline__ void qb_lds_store32(unsigned addr, unsigned v) {
  *reinterpret_cast<__attribute__((address_space(3))) unsigned*>(static_cast<uintptr_t>(addr)) = v;
}

__device__ __forceinline__ int qb_lds_load32(unsigned addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) int*>(static_cast<uintptr_t>(addr));
}

template <QpKind Q, int KB, bool MT>
__global__ void __launch_bounds__(64 * kQbWaves, 1) qi32_band_kernel(Qi32BandArgs a_in) {
  const Qi32BandArgs a = preload_args(a_in);
  const int NT = MT ? a.NT : 1;
  const int WPT = kQbWaves / NT;
  constexpr unsigned kOff = Q == kQpU8 ? 128u : 0u;
  constexpr int kKdim = 64 * KB;
  extern __shared__ v4i smem[];
  v4i* filt = smem;
  v4i* halo = smem + a.halo_lds / 16;
  int* csum = reinterpret_cast<int*>(halo + (a.ni + 1) * 64);  // per unit column: sum of its 64 values
  int* tsum = csum + a.ni * 16;                                 // per workgroup channel: filter row sum
  int* marks = tsum + NT * 64;                                  // per wave: a value outside int8
  const unsigned filt_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(filt) & 0xffffffffu);
  const unsigned halo_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(halo) & 0xffffffffu);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row_l = lane & 15;
  const int grp_l = lane >> 4;

  const int lin = xcd_tile(blockIdx.x, a.nblocks);
  const int band = fdiv(lin, a.fd_ntiles);
  const int ctile = lin - band * a.ntiles;
  const int n = fdiv(band, a.fd_bpi);
  const int rem = band - n * a.bands_per_img;
  const int blk = fdiv(rem, a.fd_bpb);  // filter block (by, bx) = (blk / Bx, blk % Bx)
  const int bib = rem - blk * a.bpb;    // band within the block
  const int by = fdiv(blk, a.fd_bx);
  const int bx = blk - by * a.Bx;
  const int gi = fdiv(ctile, a.fd_ktpg);
  const int k0 = (ctile - gi * a.kt_per_group) * NT * 64;  // first channel (in group gi)
  const int ho0 = by * a.bho + bib * a.BH;
  const int wc0 = bx * a.Wb;  // first output column
  const int tw = MT ? wave / WPT : 0;
  const int wl = wave - tw * WPT;
  const int row_instr = a.NQ * a.NPB;

  // zero points: loaded first, made uniform after the first input loads are issued
  const int zx_v = qb_zero_point<Q>(a.in_qp, n);
  const int zw_v = qb_zero_point<Q>(a.f_qp, 0);
  unsigned xpad = 0;  // staged value of a padded tap: zx - offset
  bool bad = false;

  // ---- filter: the workgroup's NT tiles of int8 fragments from the prepass, contiguous,
  // by DMA (1 KB per instruction); then the range flags of its tiles' K-blocks
  const int kt64 = a.kt_per_group * NT;
  const int tile0 = (blk * (a.ntiles / a.kt_per_group) + gi) * kt64 + k0 / 64;
  {
    const __amdgpu_buffer_rsrc_t rf = make_rsrc(a.wfrag + static_cast<size_t>(tile0) * KB * 4096, NT * KB * 4096);
    for (int f = wave; f < NT * 4 * KB; f += kQbWaves) load_lds16(rf, filt + f * 64, 16u * lane, static_cast<unsigned>(f * 1024));
    const __amdgpu_buffer_rsrc_t rfl =
        make_rsrc(a.wfrag + a.flags_off + static_cast<size_t>(tile0) * KB * 4, NT * KB * 4);
    // NT * KB <= 72 flags, two per lane; those past the range read 0
    bad = (__builtin_amdgcn_raw_buffer_load_b32(rfl, 4u * static_cast<unsigned>(lane), 0, 0) |
           __builtin_amdgcn_raw_buffer_load_b32(rfl, 4u * static_cast<unsigned>(lane + 64), 0, 0)) != 0;
  }

  // ---- input rows: one 16-byte load (4 codes) per lane, 1 KB contiguous per wave instruction
  // when C/groups == 64, converted to one LDS word.  Job e: unit i = wave + 8 (e / 4), its
  // pixels 4 (e % 4) + lane / 16, channels 4 (lane % 16) .. + 3 of the unit's quad.
  const int hi0 = ho0 * a.sh - a.ph;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(a.x + static_cast<size_t>(n) * a.H * a.W * a.C + static_cast<size_t>(gi) * a.Cg,
                (a.H * a.W * a.C - gi * a.Cg) * 4);
  const int nie = a.ni > wave ? (a.ni - wave + kQbWaves - 1) / kQbWaves : 0;
  const int nj = max(4 * nie, 1);
  // jobs in flight per lane: the last pass repeats the last job's load up to kD - 1 times, which
  // costs more than a deeper queue gains (C2: 4 in flight 14.5 us, 8: 15.1 us, 16: 16.5 us)
  constexpr int kD = 4;
  v4f jv[kD];
  bool jok[kD];
  auto job_load = [&](int e, int slot) {
    const int i = wave + kQbWaves * (e >> 2);
    const int hr = fdiv(i, a.fd_rowi);
    const int rem = i - hr * row_instr;
    const int q = fdiv(rem, a.fd_npb);
    const int pb = rem - q * a.NPB;
    const int hi = hi0 + hr;
    const int col = wc0 + 16 * pb + 4 * (e & 3) + (lane >> 4) - a.pw;
    const bool ok = static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) &&
                    static_cast<unsigned>(col) < static_cast<unsigned>(a.W);
    jok[slot] = ok;
    const unsigned off = ok ? static_cast<unsigned>(((hi * a.W + col) * a.C + 64 * q + 4 * (lane & 15)) * 4) : 0u;
    jv[slot] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
  };
  auto job_store = [&](int e, int slot) {
    const int i = wave + kQbWaves * (e >> 2);
    const int pcol = 4 * (e & 3) + (lane >> 4);
    const unsigned v = qb_pack4(jv[slot], jok[slot], kOff, xpad, bad);
    qb_lds_store32(halo_addr + 16u * static_cast<unsigned>(i * 64 + 16 * ((lane & 15) >> 2) + pcol) +
                       4u * static_cast<unsigned>(lane & 3),
                   v);
  };
  // Every pass issues the same loads (indices past the end repeat the last job, whose data is
  // never used), so the compiler's waits count exactly the loads still in flight.
#pragma unroll
  for (int u = 0; u < kD; ++u) job_load(min(u, nj - 1), u);
  const int zx = __builtin_amdgcn_readfirstlane(zx_v);
  const int zw = __builtin_amdgcn_readfirstlane(zw_v);
  xpad = static_cast<unsigned>(zx) - kOff;
  for (int e0 = 0; e0 < 4 * nie; e0 += kD) {
#pragma unroll
    for (int u = 0; u < kD; ++u) {
      const int e = e0 + u;
      if (e < 4 * nie) job_store(e, u);
      job_load(min(e + kD, nj - 1), u);
    }
  }
  wait_vmcnt(0);  // the filter DMA (not tracked by the compiler)
  const bool wbad = __any(bad);
  if (lane == 0) marks[wave] = wbad ? 1 : 0;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const int band_rows = min(a.BH, a.bho - bib * a.BH);
  int any_bad = 0;
#pragma unroll
  for (int v = 0; v < kQbWaves; ++v) any_bad |= marks[v];
  any_bad = __builtin_amdgcn_readfirstlane(any_bad);
  if (any_bad) {
    // some staged value lies outside int8: direct arithmetic on the float codes for this
    // workgroup's outputs, channel fastest (the reference's loop order per output)
    const float* xn = a.x + static_cast<size_t>(n) * a.H * a.W * a.C + static_cast<size_t>(gi) * a.Cg;
    const int nk = NT * 64;
    const int nout = band_rows * a.Wb * nk;
    const int nblk = (a.bands_per_img / a.bpb);  // filter blocks
    for (int o = threadIdx.x; o < nout; o += 64 * kQbWaves) {
      const int c = o % nk;
      const int pix = o / nk;
      const int kg = k0 + c;
      if (kg >= a.Kg) continue;
      const int t = pix / a.Wb;
      const int wo = wc0 + pix - t * a.Wb;
      const int ho = ho0 + t;
      // filter [K, By, Bx, R, S, C/groups]: channel gi * Kg + kg, block blk
      const float* wk = a.w + ((static_cast<size_t>(gi) * a.Kg + kg) * nblk + blk) * kKdim;
      uint32_t acc = 0;
      for (int r = 0; r < a.R; ++r) {
        const int hi = ho * a.sh - a.ph + r * a.dh;
        if (hi < 0 || hi >= a.H) continue;
        for (int s = 0; s < a.S; ++s) {
          const int wi = wo - a.pw + s * a.dw;
          if (wi < 0 || wi >= a.W) continue;
          const float* xp = xn + (static_cast<size_t>(hi) * a.W + wi) * a.C;
          const float* wp = wk + (static_cast<size_t>(r) * a.S + s) * a.Cg;
          for (int ci = 0; ci < a.Cg; ++ci) {
            const int32_t xv = static_cast<int32_t>(xp[ci]) - zx;
            const int32_t wv = static_cast<int32_t>(wp[ci]) - zw;
            acc += static_cast<uint32_t>(xv) * static_cast<uint32_t>(wv);
          }
        }
      }
      a.y[((static_cast<size_t>(n) * a.Ho + ho) * a.Wo + wo) * a.K + static_cast<size_t>(gi) * a.Kg + kg] =
          static_cast<int32_t>(acc);
    }
    return;
  }

  // ---- filter row sums T (4 lanes per channel) and unit column sums from the staged values ----
  for (int idx = threadIdx.x; idx < NT * 256; idx += 64 * kQbWaves) {  // whole waves: the shuffles see all lanes
    const int c = idx >> 2;
    const int q = idx & 3;
    const v4i* fr = filt + ((c >> 6) * KB * 4 + ((c >> 4) & 3)) * 64 + 16 * q + (c & 15);
    int sm = 0;
#pragma unroll
    for (int b = 0; b < KB; ++b) sm += qb_bytesum(fr[b * 4 * 64]);
    sm += __shfl_xor(sm, 1);
    sm += __shfl_xor(sm, 2);
    if (q == 0) tsum[c] = sm;
  }
  for (int idx = threadIdx.x; idx < a.ni * 16; idx += 64 * kQbWaves) {
    const v4i* hc = halo + (idx >> 4) * 64 + (idx & 15);
    csum[idx] = qb_bytesum(hc[0]) + qb_bytesum(hc[16]) + qb_bytesum(hc[32]) + qb_bytesum(hc[48]);
  }

  // ---- filter registers: A[b][j] = fragment (tw, b, j) ----
  v4i A[KB][4];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) A[b][j] = filt[((tw * KB + b) * 4 + j) * 64 + lane];
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // accumulator start of this lane's channels 16j + 4 grp_l + r: dx * T + Kdim * dx * dw
  const int kt0 = k0 + 64 * tw;  // the wave's first channel (in group gi)
  const unsigned dx = kOff - static_cast<unsigned>(zx);
  const unsigned dw = kOff - static_cast<unsigned>(zw);
  const unsigned c0 = static_cast<unsigned>(kKdim) * dx * dw;
  v4i acc0[4];
  {
    const v4i* ts = reinterpret_cast<const v4i*>(tsum + 64 * tw + 4 * grp_l);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i tv = ts[4 * j];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc0[j][r] = static_cast<int>(dx * static_cast<unsigned>(tv[r]) + c0);
    }
  }
  const int nj_ok = min(4, (a.Kg - kt0) >> 4);  // 16-channel blocks of the wave inside the group

  const unsigned csum_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(csum) & 0xffffffffu);
  unsigned baddr[KB], caddr[KB];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    const int x = row_l + (a.tap[b] & 0xff);
    baddr[b] = halo_addr + 16u * static_cast<unsigned>((a.tap[b] >> 8) + 16 * grp_l + x + 48 * (x >> 4));
    // the same slot's unit column in the column sums: unit slot / 64, column x % 16
    caddr[b] = csum_addr + 4u * static_cast<unsigned>(((a.tap[b] >> 8) >> 2) + x);
  }
  const unsigned row_bytes = 16u * static_cast<unsigned>(a.sh * row_instr * 64);

  // Output: lane (pixel row_l, grp_l) stores channels 16j + 4 grp_l .. + 3 of acc[j]: the 4
  // lanes of a pixel write 64 contiguous bytes per store.
  const size_t out0 = ((static_cast<size_t>(n) * a.Ho + ho0) * a.Wo + wc0) * a.K + static_cast<size_t>(gi) * a.Kg;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y + out0, (band_rows * a.Wo - wc0) * a.K * 4);
  const unsigned lane_out = static_cast<unsigned>((row_l * a.K + kt0 + 4 * grp_l) * 4);
  const int nseg = band_rows * a.SEGR;
  int seg_t = 0, seg_c = wl;
  while (seg_c >= a.SEGR) {
    seg_c -= a.SEGR;
    ++seg_t;
  }
  unsigned seg_in = static_cast<unsigned>(seg_t) * row_bytes + 1024u * static_cast<unsigned>(seg_c);
  int seg_out = (seg_t * a.Wo + 16 * seg_c) * a.K;
  const unsigned lane_last = lane_out + (16 * (a.SEGR - 1) + row_l < a.Wb ? 0u : 0x40000000u);
  auto seg_soff = [&]() { return static_cast<unsigned>(seg_out * 4); };
  auto seg_lane = [&]() { return seg_c == a.SEGR - 1 ? lane_last : lane_out; };
  auto seg_next = [&]() {
    seg_c += a.dS;
    seg_in += static_cast<unsigned>(a.d_rb);
    seg_out += a.d_out;
    if (seg_c >= a.SEGR) {
      seg_c -= a.SEGR;
      seg_in += static_cast<unsigned>(a.c_rb);
      seg_out += a.c_out;
    }
  };
  // sum of the pixel's staged window: the column sums of its KB (tap, quad) positions
  auto window_sum = [&](unsigned rb) {
    const unsigned cb = rb >> 4;  // segment offset: 1024 halo bytes per 16 unit columns of 4 bytes
    unsigned s = 0;
#pragma unroll
    for (int b = 0; b < KB; ++b) s += static_cast<unsigned>(qb_lds_load32(caddr[b] + cb));
    return s;
  };
  auto emit = [&](const v4i (&acc)[4], unsigned wsum, unsigned soff, unsigned lane_q) {
    const unsigned corr = dw * wsum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nj_ok) {
        v4i v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = static_cast<int>(static_cast<unsigned>(acc[j][r]) + corr);
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, lane_q + 64u * j, soff, kStoreAux);
        store_gap(v);
      }
    }
  };
  auto mfma_phase = [&](unsigned rb, v4i (&acc)[4]) {
    constexpr int RS = KB < 4 ? KB : 4;
    v4i B[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) B[r] = lds_read16(baddr[r] + rb);
#pragma unroll
    for (int b = 0; b < KB; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b % RS], b == 0 ? acc0[j] : acc[j], 0, 0, 0);
      }
      if (b + RS < KB) B[b % RS] = lds_read16(baddr[b + RS] + rb);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // the two waves of a SIMD (w and w + 4) skewed by one epilogue, as in the int8 band kernel
  const int nph = wl < nseg ? (nseg - wl + WPT - 1) / WPT : 0;
  v4i acc[4];
  if (wave < kQbWaves / 2) {
    for (int p = 0; p < nph; ++p) {
      mfma_phase(seg_in, acc);
      const unsigned ws = window_sum(seg_in);
      emit(acc, ws, seg_soff(), seg_lane());
      seg_next();
    }
  } else {
    unsigned soff_prev = 0, lane_prev = 0, ws_prev = 0;
    for (int p = 0; p < nph; ++p) {
      v4i prev[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) prev[j] = acc[j];
      if (p > 0) emit(prev, ws_prev, soff_prev, lane_prev);
      mfma_phase(seg_in, acc);
      ws_prev = window_sum(seg_in);
      soff_prev = seg_soff();
      lane_prev = seg_lane();
      seg_next();
    }
    if (nph > 0) emit(acc, ws_prev, soff_prev, lane_prev);
  }
}

// Filter prepass: block (tile, b) converts K-block b (64 values of every channel) of one
// 64-channel tile of a group to offset int8 in MFMA fragment order, fragment (b, j) = channels
// 16j .. 16j + 15, lane (row, q) of it holding bytes 16q .. 16q + 15 of the K-block of channel
// 16j + row; channels past K/groups are zeros.  Thread (channel c, quarter p) converts values
// 4p + 16k, k = 0..3, so the 4 threads of a channel fill one 16-byte slot per k.  The block
// writes 1 to its range flag when a value lies outside int8.
// With blocked filters ([K, By, Bx, R, S, C/groups], nblk = By * Bx blocks) the tiles of block
// fb come after those of blocks 0 .. fb - 1: tile = (fb * G + group) * kt64 + tile in group.
template <QpKind Q>
__global__ void __launch_bounds__(256) qi32_filter_prep_kernel(const float* w, int8_t* frag, int* flags, int Kg,
                                                               int Kdim, int kt64, int KB, int G, int nblk) {
  constexpr unsigned kOff = Q == kQpU8 ? 128u : 0u;
  const int blk = blockIdx.x;
  const int tile = blk / KB;
  const int b = blk - tile * KB;
  const int gt = tile / kt64;  // fb * G + gi
  const int fb = gt / G;
  const int gi = gt - fb * G;
  const int c = threadIdx.x >> 2;
  const int p = threadIdx.x & 3;
  const int kg = 64 * (tile - gt * kt64) + c;
  const bool ok = kg < Kg;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(w + (static_cast<size_t>(gi) * Kg * nblk + fb) * Kdim, ((Kg - 1) * nblk + 1) * Kdim * 4);
  const unsigned src = static_cast<unsigned>((min(kg, Kg - 1) * nblk * Kdim + 64 * b + 4 * p) * 4);
  v4f v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rw, src + 64u * k, 0, 0));
  bool bad = false;
  unsigned* out = reinterpret_cast<unsigned*>(frag + static_cast<size_t>(tile) * KB * 4096 +
                                              16 * ((b * 4 + ((c >> 4) & 3)) * 64 + (c & 15)) + 4 * p);
#pragma unroll
  for (int k = 0; k < 4; ++k) out[64 * k] = qb_pack4(v[k], ok, kOff, 0u, bad);
  const int any = __syncthreads_or(bad ? 1 : 0);
  if (threadIdx.x == 0) flags[blk] = any ? 1 : 0;
}

struct Qi32BandPlan {
  int KB, NQ, NPB, SEGR, NT, WPT, BH, bands_per_img, kt_per_group, HR, ni;
  int halo_lds;
  size_t lds_bytes;
};

int qb_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

size_t qb_lds_bytes(int KB, int nt, long long ni) {
  return static_cast<size_t>(nt) * qb_tile_slots(KB) * 16 + static_cast<size_t>(ni + 1) * 1024 +
         static_cast<size_t>(ni) * 64 + static_cast<size_t>(nt) * 256 + 4 * kQbWaves;
}

bool qb_plan(const Geom& g, const BlockGeom& bg, Qi32BandPlan* p, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  // the workgroup's columns: a filter block's (all of them for a plain filter)
  const int Wb = bg.bwo;
  const int Hb = bg.bho;
  if (g.Cg % 64 != 0 || g.Cg == 0) return no("qi32 band kernel needs (c/groups) % 64 == 0");
  if (g.Kg <= 0 || g.Kg % 16 != 0) return no("qi32 band kernel needs (k/groups) % 16 == 0");
  if (g.sw != 1) return no("qi32 band kernel needs stride_w == 1");
  if (g.sh < 1 || g.dh < 1 || g.dw < 1 || g.ph < 0 || g.pw < 0) return no("qi32 band kernel needs positive stride/dilation");
  if (Wb > 64 || Wb < 1 || Hb < 1) return no("qi32 band kernel needs 1 <= output (block) width <= 64");
  if (g.R < 1 || g.S < 1) return no("qi32 band kernel needs a non-empty filter");
  const long long kb = static_cast<long long>(g.R) * g.S * (g.Cg / 64);
  if (kb > kQbMaxKB) return no("qi32 band kernel filter does not fit in registers (R*S*c/groups > 576)");
  const long long hcols = static_cast<long long>(Wb) + static_cast<long long>(g.S - 1) * g.dw;
  if (hcols > 128) return no("qi32 band kernel needs output width + dilated filter width <= 128");
  if (static_cast<long long>(g.Ho) * g.Wo * g.K * 4 >= (1LL << 30)) return no("qi32 band kernel needs images below 2^30 output bytes");
  if (static_cast<long long>(g.H) * g.W * g.C * 4 >= (1LL << 31)) return no("qi32 band kernel needs images below 2^31 input bytes");
  if (static_cast<long long>(g.Kg) * g.R * g.S * g.Cg * 4 >= (1LL << 31)) return no("qi32 band kernel needs group filters below 2^31 bytes");
  if (static_cast<long long>(bg.By) * bg.Bx * g.G * ((g.Kg + 63) / 64) * g.R * g.S * (g.Cg / 64) * 4096 >= (1LL << 31)) {
    return no("qi32 band kernel needs converted filters below 2^31 bytes");
  }
  p->KB = static_cast<int>(kb);
  p->NQ = g.Cg / 64;
  p->NPB = static_cast<int>((hcols + 15) / 16);
  p->SEGR = (Wb + 15) / 16;
  const int kt64 = (g.Kg + 63) / 64;
  const int cus = qb_cu_count();
  // Cost in cycles of one round of workgroups (one per CU): the two waves of the busiest
  // SIMD run KB * 4 MFMAs plus an epilogue per phase; the loads are the filter's int8
  // fragments from the prepass and every float code of the band's rows (about 25 bytes a
  // cycle per CU).
  bool found = false;
  double best = 0.0;
  for (int nt = 1; nt <= kQbWaves; nt *= 2) {
    if (kt64 % nt != 0) continue;
    const int wpt = kQbWaves / nt;
    for (int bh = 1; bh <= Hb; ++bh) {
      const long long hr = static_cast<long long>(bh - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
      const long long ni = hr * p->NQ * p->NPB;
      if (ni > kQbWaves * 16) break;
      const size_t lds = qb_lds_bytes(p->KB, nt, ni);
      if (lds > static_cast<size_t>(kQbLds)) break;
      const long long bands = static_cast<long long>(bg.By) * bg.Bx * ((Hb + bh - 1) / bh);
      const long long wgs = static_cast<long long>(g.N) * bands * g.G * (kt64 / nt);
      const long long rounds = (wgs + cus - 1) / cus;
      const long long nph = (static_cast<long long>(bh) * p->SEGR + wpt - 1) / wpt;
      const double phase = p->KB * 64.0 + 600.0;
      const double load = 3000.0 + static_cast<double>(nt * 4096LL * p->KB + ni * 4096) / 25.0;
      const double cost = static_cast<double>(rounds) * (2.0 * static_cast<double>(nph) * phase + load);
      if (!found || cost < best - 1e-9) {
        found = true;
        best = cost;
        p->NT = nt;
        p->WPT = wpt;
        p->kt_per_group = kt64 / nt;
        p->BH = bh;
        p->bands_per_img = static_cast<int>(bands);
        p->HR = static_cast<int>(hr);
        p->ni = static_cast<int>(ni);
        p->halo_lds = static_cast<int>(static_cast<size_t>(nt) * qb_tile_slots(p->KB) * 16);
        p->lds_bytes = lds;
      }
    }
  }
  if (!found) return no("qi32 band kernel input rows do not fit in LDS");
  const long long blocks = static_cast<long long>(g.N) * p->bands_per_img * g.G * p->kt_per_group;
  if (blocks > 0x7fffffffLL) return no("grid too large");
  return true;
}

template <QpKind Q, int KB>
void qb_launch(const Qi32BandArgs& a, const Qi32BandPlan& pl, unsigned nblocks, hipStream_t stream) {
  auto kern = pl.NT > 1 ? qi32_band_kernel<Q, KB, true> : qi32_band_kernel<Q, KB, false>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(pl.lds_bytes));
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(64 * kQbWaves), pl.lds_bytes, stream, a);
}

template <QpKind Q, int KB>
void qb_dispatch(int kb, const Qi32BandArgs& a, const Qi32BandPlan& pl, unsigned nblocks, hipStream_t stream) {
  if constexpr (KB >= 1) {
    if (kb == KB) {
      qb_launch<Q, KB>(a, pl, nblocks, stream);
    } else {
      qb_dispatch<Q, KB - 1>(kb, a, pl, nblocks, stream);
    }
  }
}

bool qb_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool qi32_band_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, const void* y,
                        std::string* why) {
  if (!qb_aligned16(x) || !qb_aligned16(w) || !qb_aligned16(y)) {
    if (why) *why = "qi32 band kernel needs 16-byte aligned x, w and y";
    return false;
  }
  Qi32BandPlan pl;
  return qb_plan(g, bg, &pl, why);
}

size_t qi32_band_workspace_bytes(const Geom& g, const BlockGeom& bg) {
  const size_t nfblk =
      static_cast<size_t>(bg.By) * bg.Bx * g.G * ((g.Kg + 63) / 64) * g.R * g.S * (g.Cg / 64);
  return nfblk * 4096 + nfblk * 4;
}

hipError_t launch_qi32_band(const Geom& g, const BlockGeom& bg, QpKind qp, const float* x, const float* w, int32_t* y,
                            const void* in_qp, const void* f_qp, void* ws, hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  Qi32BandPlan pl;
  if (!qb_plan(g, bg, &pl, nullptr)) return hipErrorInvalidConfiguration;
  Qi32BandArgs a;
  a.x = x; a.w = w; a.y = y;
  a.in_qp = static_cast<const unsigned char*>(in_qp);
  a.f_qp = static_cast<const unsigned char*>(f_qp);
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.sh = g.sh; a.dh = g.dh; a.dw = g.dw; a.R = g.R; a.S = g.S;
  a.Cg = g.Cg; a.Kg = g.Kg;
  a.BH = pl.BH; a.bands_per_img = pl.bands_per_img; a.NT = pl.NT;
  a.kt_per_group = pl.kt_per_group; a.NQ = pl.NQ; a.NPB = pl.NPB; a.SEGR = pl.SEGR;
  a.ni = pl.ni;
  a.halo_lds = pl.halo_lds;
  // K-block b = (tap, chunk quad): halo slot offset of its filter row and quad, column shift
  for (int b = 0; b < kQbMaxKB; ++b) {
    if (b < pl.KB) {
      const int tap = b / pl.NQ;
      const int q = b % pl.NQ;
      const int r = tap / g.S;
      const int s = tap % g.S;
      a.tap[b] = ((r * g.dh * pl.NQ + q) * pl.NPB * 64) << 8 | (s * g.dw);
    } else {
      a.tap[b] = 0;
    }
  }
  a.ntiles = g.G * pl.kt_per_group;
  a.fd_ntiles = fastdiv_m(a.ntiles);
  a.Wb = bg.bwo;
  a.bho = bg.bho;
  a.Bx = bg.Bx;
  a.bpb = (bg.bho + pl.BH - 1) / pl.BH;
  a.fd_bpb = fastdiv_m(a.bpb);
  a.fd_bx = fastdiv_m(bg.Bx);
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_ktpg = fastdiv_m(pl.kt_per_group);
  a.fd_rowi = fastdiv_m(pl.NQ * pl.NPB);
  a.fd_npb = fastdiv_m(pl.NPB);
  {
    const int dT = pl.WPT / pl.SEGR;
    const int row_bytes = g.sh * pl.NQ * pl.NPB * 1024;
    a.dS = pl.WPT % pl.SEGR;
    a.d_rb = dT * row_bytes + 1024 * a.dS;
    a.c_rb = row_bytes - 1024 * pl.SEGR;
    a.d_out = (dT * g.Wo + 16 * a.dS) * g.K;
    a.c_out = (g.Wo - 16 * pl.SEGR) * g.K;
  }
  const long long nblocks = static_cast<long long>(g.N) * pl.bands_per_img * g.G * pl.kt_per_group;
  a.nblocks = static_cast<int>(nblocks);
  // the workspace (qi32_band_workspace_bytes) holds the prepass's fragments, then its flags
  const int kt64 = (g.Kg + 63) / 64;
  const int nblk = bg.By * bg.Bx;
  const int nfblk = nblk * g.G * kt64 * pl.KB;
  const size_t frag_bytes = static_cast<size_t>(nfblk) * 4096;
  a.wfrag = static_cast<const int8_t*>(ws);
  a.flags_off = static_cast<int>(frag_bytes);
  int8_t* frag = static_cast<int8_t*>(ws);
  int* flags = reinterpret_cast<int*>(frag + frag_bytes);
  if (qp == kQpU8) {
    hipLaunchKernelGGL(qi32_filter_prep_kernel<kQpU8>, dim3(nfblk), dim3(256), 0, stream, w, frag, flags, g.Kg,
                       g.R * g.S * g.Cg, kt64, pl.KB, g.G, nblk);
    qb_dispatch<kQpU8, kQbMaxKB>(pl.KB, a, pl, static_cast<unsigned>(nblocks), stream);
  } else {
    hipLaunchKernelGGL(qi32_filter_prep_kernel<kQpS5>, dim3(nfblk), dim3(256), 0, stream, w, frag, flags, g.Kg,
                       g.R * g.S * g.Cg, kt64, pl.KB, g.G, nblk);
    qb_dispatch<kQpS5, kQbMaxKB>(pl.KB, a, pl, static_cast<unsigned>(nblocks), stream);
  }
  return hipGetLastError();
}

}  // namespace miq
