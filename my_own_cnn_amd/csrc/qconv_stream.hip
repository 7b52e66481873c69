// int8 convolution with the filter streamed through LDS (v_mfma_i32_16x16x64_i8): bands of
// whole output rows, for filters too large to keep in registers or strides the row-band
// kernel does not take (stride_w 2).  Needs (C/groups) % 64 == 0 and (K/groups) % 128 == 0.
//
// Work decomposition.  A workgroup of 8 waves (two per SIMD) owns RB output rows of one
// image, all Wo columns, and KT = 64 * WK output channels of one group (WK = 2 or 4).  The
// band's pixels are packed row-major into 16-pixel segments (a segment may run from one
// output row into the next).  Wave w computes the 64 channels of tile w % WK for segments
// w / WK, w / WK + WP, ... (WP = 8 / WK waves per tile, at most 4 segments each).
//
// Input rows.  The band's HR = (RB - 1) * sh + (R - 1) * dh + 1 input rows go to LDS, row
// after row, each as [chunk quad][column parity][16-column block][chunk in quad][column in
// block] x 16 bytes (a chunk is 16 channels, a quad 4 chunks).  Halo column hc (input
// column hc - pw) has parity hc % sw and position hc / sw in its parity plane, so the B
// fragment of tap (r, s) for output column wo reads parity plane (s * dw) % sw at position
// wo + (s * dw) / sw: the 16 lanes of a lane group (16 consecutive pixels of one row) read
// consecutive slots, free of bank conflicts.  Rows are RowS slots apart, padded so that
// sh * RowS = Wo (mod 16): a segment that runs into the next output row keeps 16 distinct
// slots modulo 16.  One buffer_load_dwordx4 ... lds (global -> LDS, no registers) fills one
// (row, quad, parity, block): 16 pixels x 64 channel bytes.  The buffer range check turns
// padding into zeros (an out-of-image row or column gets an offset past num_records).
//
// Filter.  K-block b (tap b / NQ, chunk quad b % NQ; NQ = Cg / 64) of the workgroup's KT
// channels is 4 * WK fragments of 1 KB (64-channel tile t, MFMA row block j; lane l's 16
// bytes at l * 16), one load instruction each.  K-blocks stream through a ring of D
// buffers.  The K-loop is software-pipelined: while the MFMAs of K-block b run from
// registers, the fragments of K-block b + 1 are read from LDS.  Before those reads a wave
// waits for its own loads of b + 1 (loads complete in order and no store is issued before
// the epilogue, so the count is exact) and a barrier publishes every wave's; the same
// barrier shows that every wave has read K-block b into its registers, so b's buffer then
// receives K-block b + D.
//
// int8 outputs permute channels as in the other MFMA kernels (MFMA j row rho <-> channel
// 16 * (rho / 4) + 4j + rho % 4), so each lane holds 16 consecutive channels of one pixel;
// 4-byte outputs keep the natural order (channel 16j + rho).
// Accumulators start at the bias; the epilogue is the shared int8 arithmetic and one
// 16-byte non-temporal store per lane (four for int32 / fp32 outputs), each followed by
// store_gap() on its data registers.

#include "qconv_device.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace miq {
namespace {

constexpr int kStreamWaves = 8;
constexpr int kStreamNseg = 4;  // segments per wave at most
constexpr int kStreamLds = 160 * 1024;
constexpr int kStreamMaxRing = 6;  // ring depths 3 .. 6 are instantiated

struct StreamArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  void* y;
  int H, W, C, K, Ho, Wo;
  int ph, pw, sh, sw, dh, dw;
  int S, Cg, Kg, Kdim;
  int RB;             // output rows per band
  int bands_per_img;  // ceil(Ho / RB)
  int kt_per_group;   // workgroup channel tiles (KT channels) per group
  int nblocks;        // workgroups of the launch
  int NQ, NPB;        // chunk quads per tap (Cg / 64), 16-column blocks per parity plane
  int RowS;           // LDS slots (16 bytes) per input row, padded
  int KB;             // K-blocks
  int ni;             // input load instructions per workgroup: HR * NQ * sw * NPB
  int ring_lds, ep_lds, halo_lds;  // LDS byte offsets
  float act_scale;
  int relu;
  int ntiles;         // workgroup channel tiles per band: groups * kt_per_group
  FastDivM fd_wo, fd_ntiles, fd_bpi, fd_ktpg, fd_rowi, fd_npb, fd_sw;
};

static_assert(sizeof(StreamArgs) <= 256, "kernel arguments fit one s_load batch");

// Calls f(std::integral_constant<int, n>) for a wave-uniform 0 <= n <= NMAX: one
// branch-free instantiation of the callee per count.
template <int NMAX, typename F>
__device__ __forceinline__ void dispatch_count_z(int n, F&& f) {
  if constexpr (NMAX > 0) {
    if (n == NMAX) {
      f(std::integral_constant<int, NMAX>{});
    } else {
      dispatch_count_z<NMAX - 1>(n, f);
    }
  } else {
    f(std::integral_constant<int, 0>{});
  }
}

// s_waitcnt vmcnt(n) lgkmcnt(0), n <= 15, as the builtin: the compiler's own wait
// insertion then knows that every LDS read issued before it has completed.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N <= 15, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x70 | N);
}

template <int WK, int EPI, int D>
__global__ void __launch_bounds__(64 * kStreamWaves, 1) i8_stream_kernel(StreamArgs a_in) {
  const StreamArgs a = preload_args(a_in);
  // 4-byte outputs use natural channel order (MFMA row block j, row rho <-> channel 16j + rho),
  // so the 4 lanes of a pixel store 64 contiguous bytes per instruction; int8 outputs keep 16
  // consecutive channels per lane (one 16-byte store).
  constexpr bool NAT = EPI != kEpiI8;
  constexpr int WP = kStreamWaves / WK;  // waves per 64-channel tile
  constexpr int LPW = WK / 2;            // filter loads per wave per K-block (4 * WK over 8 waves)
  extern __shared__ v4i st_lds[];
  v4i* ring = st_lds + a.ring_lds / 16;
  v4i* halo = st_lds + a.halo_lds / 16;
  v4i* ep = st_lds + a.ep_lds / 16;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row_l = lane & 15;
  const int grp_l = lane >> 4;
  const int wk = wave % WK;
  const int wp = wave / WK;

  const int lin = xcd_tile(blockIdx.x, a.nblocks);
  const int band = fdiv(lin, a.fd_ntiles);
  const int ctile = lin - band * a.ntiles;
  const int n = fdiv(band, a.fd_bpi);
  const int bi = band - n * a.bands_per_img;
  const int gi = fdiv(ctile, a.fd_ktpg);
  const int kwg0 = (ctile - gi * a.kt_per_group) * (64 * WK);  // first channel (in group gi)
  const int ho0 = bi * a.RB;
  const int rows = min(a.RB, a.Ho - ho0);


  // ---- input rows: instruction i = ((hr * NQ + q) * sw + par) * NPB + pb to wave i % 8;
  // lane l reads parity-plane position 16 * pb + l % 16 (halo column * sw + par), chunk
  // 4q + l / 16.  Rows and columns outside the image get 2^30: past num_records.
  {
    const int hi0 = ho0 * a.sh - a.ph;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + static_cast<size_t>(n) * a.H * a.W * a.C, a.H * a.W * a.C);
    const int row_instr = a.NQ * a.sw * a.NPB;
    for (int i = wave; i < a.ni; i += kStreamWaves) {
      const int hr = fdiv(i, a.fd_rowi);
      const int rem = i - hr * row_instr;
      const int qp = fdiv(rem, a.fd_npb);
      const int pb = rem - qp * a.NPB;
      const int q = fdiv(qp, a.fd_sw);
      const int par = qp - q * a.sw;
      const int hi = hi0 + hr;
      const unsigned soff = static_cast<unsigned>(hi) < static_cast<unsigned>(a.H)
                                ? static_cast<unsigned>((hi * a.W) * a.C + gi * a.Cg + 64 * q)
                                : 0x40000000u;
      const int wi = (16 * pb + row_l) * a.sw + par - a.pw;
      const unsigned voff =
          static_cast<unsigned>(wi) < static_cast<unsigned>(a.W) ? static_cast<unsigned>(wi * a.C + 16 * grp_l) : 0x40000000u;
      load_lds16(rx, halo + hr * a.RowS + rem * 64, voff, soff);
    }
  }
  // ---- bias (wave 0) and per-channel scales (wave 1) of the KT channels: 1 KB each.
  // kEpiQi32: the filter row sums T (in bias) and image n's 16-byte record {dx, dw,
  // Kdim * dx * dw, 0} (in wscale) ----
  if (EPI != kEpiAcc32 && wave < 2) {
    const int valid = max(0, a.Kg - kwg0) * 4;
    const size_t off = static_cast<size_t>(gi) * a.Kg + kwg0;
    if (wave == 0) {
      load_lds16(make_rsrc(a.bias ? a.bias + off : nullptr, a.bias ? valid : 0), ep, 16u * lane, 0);
    } else if constexpr (EPI == kEpiQi32) {
      load_lds16(make_rsrc(a.wscale + 4 * static_cast<size_t>(n), 16), ep + 64, 16u * lane, 0);
    } else {
      load_lds16(make_rsrc(a.wscale + off, valid), ep + 64, 16u * lane, 0);
    }
  }
  // ---- filter K-blocks: fragment f = 4t + j of K-block b is one instruction, to wave f % 8;
  // its lane (row_l, grp_l) reads channel kwg0 + 64t + 16 * (row_l / 4) + 4j + row_l % 4,
  // bytes [64b + 16 * grp_l, +16) of that channel's KRSC row (K-block b = tap * NQ + q covers
  // row bytes tap * Cg + 64q = 64b).
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(gi) * a.Kg * a.Kdim, a.Kg * a.Kdim);
  const unsigned lane_row =
      static_cast<unsigned>((NAT ? row_l : 16 * (row_l >> 2) + (row_l & 3)) * a.Kdim + 16 * grp_l);
  auto issue_filter = [&](int b, int slot) {  // K-block b into ring buffer `slot`
    v4i* buf = ring + slot * (4 * WK * 64);
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const int f = wave + kStreamWaves * u;
      const int t = f >> 2;
      const int j = f & 3;
      load_lds16(rw, buf + f * 64, lane_row, static_cast<unsigned>((kwg0 + 64 * t + (NAT ? 16 : 4) * j) * a.Kdim + 64 * b));
    }
  };
  const int pre = min(D, a.KB);
  for (int b = 0; b < pre; ++b) issue_filter(b, b);

  // per segment i of this wave: packed pixel p = 16 * (wp + i * WP) + row_l of the band,
  // output row lho = p / Wo, column lwo = p % Wo; pixels outside the band read row 0 /
  // column 0 (finite data, never stored)
  int lwo[kStreamNseg], rbase[kStreamNseg];
  unsigned ovoff[kStreamNseg];
  const int nseg_band = (rows * a.Wo + 15) >> 4;
  const int nsv = min(kStreamNseg, max(0, (nseg_band - wp + WP - 1) / WP));
  constexpr int kOutBytes = EPI == kEpiI8 ? 1 : 4;
  // this lane's first output channel (in group gi): 16 consecutive ones, or in natural order
  // channels kc0 + 16j + r
  const int kc0 = kwg0 + 64 * wk + (NAT ? 4 : 16) * grp_l;
#pragma unroll
  for (int i = 0; i < kStreamNseg; ++i) {
    const int p = 16 * (wp + i * WP) + row_l;
    const int lho = fdiv(p, a.fd_wo);
    const bool ok = lho < rows;
    lwo[i] = ok ? p - lho * a.Wo : 0;
    rbase[i] = ok ? lho * a.sh * a.RowS : 0;
    ovoff[i] = static_cast<unsigned>((p * a.K + kc0) * kOutBytes) + (ok ? 0u : 0x40000000u);
  }
  const unsigned halo_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(halo) & 0xffffffffu);
  const unsigned ring_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(ring) & 0xffffffffu);

  // Loads of K-block c (and everything issued before it) are in on every wave; the
  // barrier also ends every wave's reads of the K-block before c.  In steady state this
  // wave's loads issued after c's are those of the next D - 2 K-blocks (D - 1 after the
  // prologue); near the end fewer are, and the wait takes all (they are old by then).
  if (a.KB >= D) {
    wait_vm_lgkm0<(D - 1) * LPW>();
  } else {
    wait_vm_lgkm0<0>();
  }
  barrier_only();

  // epilogue parameters of this lane's 16 channels (kc0 + 4j + r, or kc0 + 16j + r)
  v4i bias_v[4];
  v4f mult_v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bias_v[j] = v4i{0, 0, 0, 0};
    mult_v[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EPI == kEpiI8 || EPI == kEpiF32) {
      const int ev = NAT ? 4 * j + grp_l : 4 * grp_l + j;
      bias_v[j] = ep[16 * wk + ev];
      const v4i ws = ep[64 + 16 * wk + ev];
#pragma unroll
      for (int r = 0; r < 4; ++r) mult_v[j][r] = requant_multiplier(a.act_scale, __int_as_float(ws[r]));
    }
  }
  // kEpiQi32: accumulators start at dx * T + Kdim * dx * dw; the epilogue adds dw * W(p)
  unsigned qdw = 0;
  if constexpr (EPI == kEpiQi32) {
    const v4i rec = ep[64];
    const unsigned dx = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(rec[0]));
    qdw = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(rec[1]));
    const unsigned c0 = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(rec[2]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i tv = ep[16 * wk + 4 * j + grp_l];  // natural order: channels 16j + 4 grp_l + r
#pragma unroll
      for (int r = 0; r < 4; ++r) bias_v[j][r] = static_cast<int>(dx * static_cast<unsigned>(tv[r]) + c0);
    }
  }

  // K-loop over K-blocks b = (r * S + s) * NQ + q (taps (r, s), chunk quads q), two per
  // pass so the fragment registers alternate without copies.  NS = the wave's segment
  // count (0 .. 4): a wave without segments still loads and synchronises.
  v4i acc[4][kStreamNseg];
  int wsum[kStreamNseg];  // kEpiQi32: this lane's share of each segment pixel's window sum
  auto kloop = [&](auto ns_tag) {
    constexpr int NS = decltype(ns_tag)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < kStreamNseg; ++i) acc[j][i] = bias_v[j];
#pragma unroll
    for (int i = 0; i < kStreamNseg; ++i) wsum[i] = 0;
    // tap and quad of the K-block whose fragments are read next, and each segment's slot
    // (quad 0) for that tap
    int q = 0, s = 0, tap_row = 0;  // tap_row = r * dh * RowS
    unsigned baddr[kStreamNseg > 0 ? kStreamNseg : 1];
    auto tap_addrs = [&]() {
      const int sdw = s * a.dw;
      const int sft = fdiv(sdw, a.fd_sw);
      const int par = sdw - sft * a.sw;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int x = lwo[i] + sft;
        baddr[i] = halo_addr + 16u * static_cast<unsigned>(rbase[i] + tap_row + par * a.NPB * 64 + x + 48 * (x >> 4) +
                                                           16 * grp_l);
      }
    };
    auto advance = [&]() {
      if (++q == a.NQ) {
        q = 0;
        if (++s == a.S) {
          s = 0;
          tap_row += a.dh * a.RowS;
        }
        tap_addrs();
      }
    };
    auto read_frags = [&](int rslot, v4i (&A)[4], v4i (&B)[NS > 0 ? NS : 1]) {  // from ring buffer rslot
      if constexpr (NS > 0) {
        const unsigned aaddr = ring_addr + 16u * static_cast<unsigned>(rslot * (4 * WK * 64) + (4 * wk) * 64 + lane);
        const unsigned qoff = 16u * static_cast<unsigned>(q * a.sw * a.NPB * 64);
#pragma unroll
        for (int j = 0; j < 4; ++j) A[j] = lds_read16(aaddr + 1024u * j);
#pragma unroll
        for (int i = 0; i < NS; ++i) B[i] = lds_read16(baddr[i] + qoff);
      }
    };
    auto mma = [&](const v4i (&A)[4], const v4i (&B)[NS > 0 ? NS : 1]) {
      if constexpr (NS > 0) {
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j], B[i], acc[j][i], 0, 0, 0);
        if constexpr (EPI == kEpiQi32) {
#pragma unroll
          for (int i = 0; i < NS; ++i)
#pragma unroll
            for (int d = 0; d < 4; ++d) wsum[i] = __builtin_amdgcn_sdot4(B[i][d], 0x01010101, wsum[i], false);
        }
      }
    };
    // step b: K-block b's fragments are in registers; publish b + 1, refill b's buffer
    // (slot) with b + D, read b + 1's fragments, then run b's MFMAs
    int slot = 0;  // ring buffer of K-block b: b % D
    auto next = [&](int b, v4i (&A)[4], v4i (&B)[NS > 0 ? NS : 1]) {
      if (b + D <= a.KB) {
        wait_vm_lgkm0<(D - 2) * LPW>();
      } else {
        wait_vm_lgkm0<0>();
      }
      barrier_only();
      if (b + D < a.KB) issue_filter(b + D, slot);
      slot = slot + 1 == D ? 0 : slot + 1;
      read_frags(slot, A, B);
      advance();
    };
    v4i A0[4], A1[4], B0[NS > 0 ? NS : 1], B1[NS > 0 ? NS : 1];
    tap_addrs();
    read_frags(0, A0, B0);
    advance();
    // both steps of a pass unconditional, so the compiler sees no path on which the
    // fragments about to be multiplied are still being read
    int b = 0;
    for (; b + 2 < a.KB; b += 2) {
      next(b, A1, B1);
      mma(A0, B0);
      next(b + 1, A0, B0);
      mma(A1, B1);
    }
    if (b + 1 < a.KB) {
      next(b, A1, B1);
      mma(A0, B0);
      mma(A1, B1);
    } else {
      mma(A0, B0);
    }
  };
  dispatch_count_z<kStreamNseg>(nsv, kloop);

  // ---- epilogue: one buffer resource over the band's output rows of image n, group gi ----
  const size_t out0 = (static_cast<size_t>(n) * a.Ho + ho0) * a.Wo * a.K + static_cast<size_t>(gi) * a.Kg;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(static_cast<char*>(a.y) + out0 * kOutBytes, rows * a.Wo * a.K * kOutBytes);
  const float lo = a.relu ? 0.0f : -128.0f;
#pragma unroll
  for (int i = 0; i < kStreamNseg; ++i) {
    if (i >= nsv) break;
    v4i v4[4] = {acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
    if constexpr (EPI == kEpiQi32) {
      // the pixel's window sum: the 4 lanes of its row each summed their 16 channels of every K-block
      int ws = wsum[i];
      ws += __shfl_xor(ws, 16);
      ws += __shfl_xor(ws, 32);
      const unsigned corr = qdw * static_cast<unsigned>(ws);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4i v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = static_cast<int>(static_cast<unsigned>(v4[j][r]) + corr);
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, ovoff[i] + 64u * j, 0, kStoreAux);
        store_gap(v);
      }
    } else if constexpr (EPI == kEpiI8) {
      const v4i pk = a.relu ? pack_u8_relu(v4, mult_v) : pack_i8(v4, mult_v, lo);
      __builtin_amdgcn_raw_buffer_store_b128(pk, ry, ovoff[i], 0, kStoreAux);
      store_gap(pk);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4i v = v4[j];
        if constexpr (EPI == kEpiF32) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float f = static_cast<float>(v4[j][r]) * mult_v[j][r];
            if (a.relu) f = (f > 0.0f) ? f : 0.0f;  // NaN and -0 -> +0
            v[r] = __float_as_int(f);
          }
        }
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, ovoff[i] + (NAT ? 64u : 16u) * j, 0, kStoreAux);
        store_gap(v);
      }
    }
  }
}

struct StreamPlan {
  int WK, RB, bands_per_img, kt_per_group, NQ, NPB, RowS, HR, KB, D, ni;
  int ring_lds, ep_lds, halo_lds;
  size_t lds_bytes;
};

int stream_cu_count() {
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

// Row padding p (slots) with sh * (RowS0 + p) = Wo (mod 16), RowS0 a multiple of 64; 0 when
// no p exists (then a segment that wraps rows may see 2-way bank conflicts).
int row_pad(int sh, int Wo) {
  for (int p = 0; p < 16; ++p)
    if ((sh * p - Wo) % 16 == 0) return p;
  return 0;
}

bool stream_plan(const Geom& g, Epi epi, StreamPlan* p, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  (void)epi;
  if (g.Cg % 64 != 0) return no("stream kernel needs (c/groups) % 64 == 0");
  if (g.Kg % 128 != 0) return no("stream kernel needs (k/groups) % 128 == 0");
  if (g.R < 1 || g.S < 1) return no("stream kernel needs a non-empty filter");
  // the tap walk divides s * dilation_w by the stride and indexes LDS rows with r * dilation_h
  if (g.sh < 1 || g.sw < 1 || g.dh < 1 || g.dw < 1) return no("stream kernel needs stride and dilation >= 1");
  if (g.ph < 0 || g.pw < 0) return no("stream kernel needs non-negative padding");
  if (g.sw > 4 || (g.S - 1) * g.dw / g.sw > 16) return no("stream kernel needs stride_w <= 4 and a narrow dilated filter");
  const long long kdim = static_cast<long long>(g.R) * g.S * g.Cg;
  if (static_cast<long long>(g.H) * g.W * g.C >= (1LL << 30)) return no("stream kernel needs images below 2^30 bytes");
  if (static_cast<long long>(g.Kg) * kdim >= (1LL << 30)) return no("stream kernel needs group filters below 2^30 bytes");
  if (static_cast<long long>(g.Ho) * g.Wo * g.K * 4 >= (1LL << 30)) return no("stream kernel needs images below 2^30 output bytes");
  p->NQ = g.Cg / 64;
  p->KB = static_cast<int>(kdim / 64);
  const long long hc = static_cast<long long>(g.Wo - 1) * g.sw + static_cast<long long>(g.S - 1) * g.dw + 1;
  const long long hcs = (hc + g.sw - 1) / g.sw;
  p->NPB = static_cast<int>((hcs + 15) / 16);
  const long long rows0 = static_cast<long long>(p->NQ) * g.sw * p->NPB * 64;
  if (rows0 * 16 > kStreamLds / 2) return no("stream kernel input rows do not fit in LDS");
  p->RowS = static_cast<int>(rows0) + row_pad(g.sh, g.Wo);
  const int cus = stream_cu_count();
  // Cost in cycles of a workgroup: its loads (input rows and the whole filter of its
  // channels) at about 15 bytes a cycle, or its MFMAs (two waves per SIMD, 16 cycles
  // each), whichever is longer, plus a fixed start-up and an epilogue per segment; times
  // the rounds of workgroups over the CUs.
  bool found = false;
  double best = 0.0;
  for (int wk = 4; wk >= 2; wk /= 2) {
    if (g.Kg % (64 * wk) != 0) continue;
    const int wpt = kStreamWaves / wk;
    const size_t ring_unit = static_cast<size_t>(wk) * 4 * 1024;
    for (int rb = 1; rb <= g.Ho; ++rb) {
      const long long nseg = (static_cast<long long>(rb) * g.Wo + 15) / 16;
      const long long nsv = (nseg + wpt - 1) / wpt;
      if (nsv > kStreamNseg) break;
      const long long hr = static_cast<long long>(rb - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
      const size_t halo = static_cast<size_t>(hr) * p->RowS * 16;
      const size_t fixed = halo + 2048;
      if (fixed + 3 * ring_unit > static_cast<size_t>(kStreamLds)) break;
      const int d = static_cast<int>(std::min<size_t>(kStreamMaxRing, (kStreamLds - fixed) / ring_unit));
      const long long wgs = static_cast<long long>(g.N) * ((g.Ho + rb - 1) / rb) * g.G * (g.Kg / (64 * wk));
      const long long rounds = (wgs + cus - 1) / cus;
      const double load = (static_cast<double>(halo) + static_cast<double>(p->KB) * ring_unit) / 15.0;
      const double mfma = static_cast<double>(p->KB) * 2.0 * 4.0 * static_cast<double>(nsv) * 16.0;
      const double cost = static_cast<double>(rounds) * (std::max(load, mfma) + 3000.0 + 600.0 * static_cast<double>(nsv));
      if (!found || cost < best - 1e-9) {
        found = true;
        best = cost;
        p->WK = wk;
        p->RB = rb;
        p->bands_per_img = (g.Ho + rb - 1) / rb;
        p->kt_per_group = g.Kg / (64 * wk);
        p->HR = static_cast<int>(hr);
        p->D = d;
        p->ni = static_cast<int>(hr * p->NQ * g.sw * p->NPB);
        p->halo_lds = 0;
        p->ring_lds = static_cast<int>(halo);
        p->ep_lds = static_cast<int>(halo + static_cast<size_t>(d) * ring_unit);
        p->lds_bytes = fixed + static_cast<size_t>(d) * ring_unit;
      }
    }
  }
  if (!found) return no("stream kernel input rows do not fit in LDS");
  const long long blocks = static_cast<long long>(g.N) * p->bands_per_img * g.G * p->kt_per_group;
  if (blocks > 0x7fffffffLL) return no("grid too large");
  return true;
}

template <int WK, int D>
void stream_launch(const StreamArgs& a, const StreamPlan& pl, Epi epi, unsigned nblocks, hipStream_t stream) {
  auto go = [&](auto kern) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(pl.lds_bytes));
    hipLaunchKernelGGL(kern, dim3(nblocks), dim3(64 * kStreamWaves), pl.lds_bytes, stream, a);
  };
  switch (epi) {
    case kEpiI8: go(i8_stream_kernel<WK, kEpiI8, D>); break;
    case kEpiAcc32: go(i8_stream_kernel<WK, kEpiAcc32, D>); break;
    case kEpiQi32: go(i8_stream_kernel<WK, kEpiQi32, D>); break;
    default: go(i8_stream_kernel<WK, kEpiF32, D>); break;
  }
}

template <int WK>
void stream_launch_d(const StreamArgs& a, const StreamPlan& pl, Epi epi, unsigned nblocks, hipStream_t stream) {
  switch (pl.D) {
    case 3: stream_launch<WK, 3>(a, pl, epi, nblocks, stream); break;
    case 4: stream_launch<WK, 4>(a, pl, epi, nblocks, stream); break;
    case 5: stream_launch<WK, 5>(a, pl, epi, nblocks, stream); break;
    default: stream_launch<WK, 6>(a, pl, epi, nblocks, stream); break;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool stream_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                     std::string* why) {
  const bool params_ok = epi == kEpiAcc32 || ((rq.bias == nullptr || aligned16(rq.bias)) && aligned16(rq.wscale));
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || !params_ok) {
    if (why) *why = "stream kernel needs 16-byte aligned tensors, bias and scales";
    return false;
  }
  StreamPlan pl;
  return stream_plan(g, epi, &pl, why);
}

namespace {

hipError_t launch_stream_any(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                             hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  StreamPlan pl;
  if (!stream_plan(g, epi, &pl, nullptr)) return hipErrorInvalidConfiguration;
  StreamArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.sh = g.sh; a.sw = g.sw; a.dh = g.dh; a.dw = g.dw;
  a.S = g.S; a.Cg = g.Cg; a.Kg = g.Kg; a.Kdim = g.R * g.S * g.Cg;
  a.RB = pl.RB; a.bands_per_img = pl.bands_per_img; a.kt_per_group = pl.kt_per_group;
  a.NQ = pl.NQ; a.NPB = pl.NPB; a.RowS = pl.RowS; a.KB = pl.KB; a.ni = pl.ni;
  a.ring_lds = pl.ring_lds; a.ep_lds = pl.ep_lds; a.halo_lds = pl.halo_lds;
  a.act_scale = rq.act_scale; a.relu = rq.relu;
  a.ntiles = g.G * pl.kt_per_group;
  a.fd_wo = fastdiv_m(g.Wo);
  a.fd_ntiles = fastdiv_m(a.ntiles);
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_ktpg = fastdiv_m(pl.kt_per_group);
  a.fd_rowi = fastdiv_m(pl.NQ * g.sw * pl.NPB);
  a.fd_npb = fastdiv_m(pl.NPB);
  a.fd_sw = fastdiv_m(g.sw);
  const long long nblocks = static_cast<long long>(g.N) * pl.bands_per_img * g.G * pl.kt_per_group;
  a.nblocks = static_cast<int>(nblocks);
  if (pl.WK == 4) {
    stream_launch_d<4>(a, pl, epi, static_cast<unsigned>(nblocks), stream);
  } else {
    stream_launch_d<2>(a, pl, epi, static_cast<unsigned>(nblocks), stream);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_i8_stream(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                            hipStream_t stream) {
  return launch_stream_any(g, epi, x, w, y, rq, stream);
}

hipError_t launch_i8_stream_qi32(const Geom& g, const int8_t* x, const int8_t* w, const int32_t* T,
                                 const int32_t* qrec, int32_t* y, hipStream_t stream) {
  const Requant rq{T, reinterpret_cast<const float*>(qrec), 1.0f, 0};
  return launch_stream_any(g, kEpiQi32, x, w, y, rq, stream);
}

}  // namespace miq
