// int8 convolution for stride-1 layers whose filter fits in registers (R*S*C/groups <= 576):
// row bands enumerated as "virtual" pixels, filter-stationary v_mfma_i32_16x16x64_i8, and
// each segment's requantization spread through the next segment's matrix instructions.
//
// Virtual pixels.  A band of bh output rows of one image reads HR = bh + (R-1)*dh input rows
// (stride 1).  Its input halo sits in LDS as a flat sequence of HR rows of L = Wo + (S-1)*dw
// columns (halo column x holds input column x - pw, zero outside the image), and output
// pixel (t, c) of the band is virtual pixel v = t*L + c.  For tap (r, s) that pixel reads
// halo pixel v + r*dh*L + s*dw: one fixed shift per tap, whatever the row.  Output pixels are
// cut into segments of 16 consecutive virtual pixels; the L - Wo columns past each row's end
// are computed and dropped (ResNet-50 3x3: 2 of 58, where segments aligned to output rows
// would drop 8 of 64).
//
// LDS layout of the halo: [chunk quad][16-pixel block][chunk in quad][pixel in block] x 16 B
// (a chunk is 16 channels, a quad 64).  One buffer_load_dwordx4 ... lds (global -> LDS, no
// registers) fills one (quad, block): its 64 lanes read 16 consecutive virtual pixels x 64
// channel bytes, one or two contiguous runs of NHWC input; pixels outside the image get an
// offset past num_records and read zero.  Lane (i, g) of an MFMA B fragment (pixel i of the
// segment, chunk g of the K-block's quad) reads virtual pixel u = 16*seg + i + shift, whose
// 16-byte slot is block(u)*64 + g*16 + u%16: the 16 pixels of a lane group hit 16 distinct
// slots modulo 16 (no bank conflicts), and the address is a per-lane constant per K-block
// plus 1024*seg.
//
// Work.  A workgroup of 8 waves (two per SIMD: wave w on SIMD w%4, h = w/4) owns one band
// and one 64-channel tile; each wave keeps the tile's whole filter in registers (KB K-blocks
// x 4 MFMA row blocks of 16 bytes per lane).  With nseg segments, M = nseg/4 "main" segments
// go to each SIMD (segment s + 4k to SIMD s, alternating between its two waves), and the
// T = nseg%4 tail segments are split by 16-channel block so that every SIMD does the same
// number of matrix instructions: tail segment j, channel block b goes to SIMD b, wave j%2.
// A tail chain is one 16x16 output block (9 MFMAs for a 3x3x64 filter) instead of a whole
// segment (36).  Three tail segments are rounded up to one more main segment (a junk one).
//
// Phases.  A wave computes one main segment per phase (4 independent accumulator chains)
// and, in its last phase, its tail chain.  The requantization of the previous phase's
// segment (16 values per lane: convert, scale, clamp, round/pack) is spread evenly over the
// current phase's K-blocks, and its 16-byte store goes out when its last value is packed, so
// the VALU work issues between matrix instructions of this wave and of the SIMD's other
// wave.  Accumulators start at the bias (read from LDS at the phase start).
//
// Loads and synchronisation.  Every load is issued at the start, spread round-robin over
// the 8 waves: first the halo blocks that phase 0 reads, then the filter, the bias and the
// scales, then the rest of the halo.  A wave waits (vmcnt) for its share of the first group
// and a barrier publishes it; after phase 0's matrix instructions every wave waits for all
// its loads and a second barrier publishes the rest of the halo.  Both waits are exact: no
// store is issued before the second barrier.  All waves execute both barriers.
//
// Filter in LDS.  With an odd K-block count the tile's 64 KRSC rows (4*KB kilobytes) are
// loaded as they lie, 1 KB per instruction, channels 32..63 shifted 32 bytes further on; the
// fragment reads (channel 16*(i/4) + 4*j + i%4 in lane row i) then meet every ds_read_b128
// cycle's 16 lanes in 16 distinct slots modulo 16.  With an even count the fragments are
// loaded in fragment order (lane l of fragment (b, j) at slot 64*(4b + j) + l).

#include "qconv_device.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace miq {
namespace {

constexpr int kFlatWaves = 8;
constexpr int kFlatMaxKB = 9;
constexpr int kFlatLds = 160 * 1024;

struct FlatArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  void* y;
  int H, W, C, K, Ho, Wo;
  int ph, pw;
  int Cg, Kg, Kdim;
  int L;              // virtual row length (halo columns): Wo + (S-1)*dw
  int rext;           // (R-1)*dh: input rows of a band beyond its output rows
  int vmax;           // largest tap shift: rext*L + (S-1)*dw
  int BH;             // output rows per band
  int bands_per_img;  // ceil(Ho / BH)
  int ktpg;           // 64-channel tiles per group
  int ntiles;         // groups * ktpg
  int nblocks;        // workgroups of the launch
  int NQ;             // chunk quads per input pixel: Cg / 64
  int qblocks;        // 16-pixel blocks per quad plane of the halo in LDS
  int filt_lds, ep_lds, halo_lds;  // LDS byte offsets
  float act_scale;
  int relu;
  // per K-block: quad << 24 | virtual shift (r*dh*L + s*dw)
  int tap[kFlatMaxKB];
  FastDivM fd_ntiles, fd_bpi, fd_ktpg, fd_L;
};

static_assert(sizeof(FlatArgs) <= 256, "kernel arguments fit one s_load batch");

__host__ __device__ constexpr int flat_filter_bytes(int KB) { return 4 * KB * 1024 + ((KB & 1) ? 64 : 0); }

template <int KB, int EPI, bool RELU>
__global__ void __launch_bounds__(64 * kFlatWaves, 1) i8_flat_kernel(FlatArgs a_in) {
  const FlatArgs a = preload_args(a_in);
  extern __shared__ v4i smem[];
  v4i* filt = smem + a.filt_lds / 16;
  v4i* ep = smem + a.ep_lds / 16;
  v4i* halo = smem + a.halo_lds / 16;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int simd = wave & 3;
  const int hh = wave >> 2;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // ---- band and channel tile (the tiles of one band are neighbours: one XCD's L2) ----
  const int lin = xcd_tile(blockIdx.x, a.nblocks);
  const int band = fdiv(lin, a.fd_ntiles);
  const int ctile = lin - band * a.ntiles;
  const int n = fdiv(band, a.fd_bpi);
  const int bi = band - n * a.bands_per_img;
  const int gi = fdiv(ctile, a.fd_ktpg);
  const int k0 = (ctile - gi * a.ktpg) * 64;  // first channel of the tile in group gi
  const int ho0 = bi * a.BH;
  const int bh = min(a.BH, a.Ho - ho0);
  const int HR = bh + a.rext;
  const int P = (bh - 1) * a.L + a.Wo;  // virtual pixels up to the band's last output pixel
  const int nseg = (P + 15) >> 4;
  int M = nseg >> 2;
  int T = nseg & 3;
  if (T == 3) {  // one more main segment per SIMD (the last one past P) costs no more
    ++M;
    T = 0;
  }
  const int nmain = 4 * M;
  const int Mw = (M - hh + 1) >> 1;  // main segments of this wave: simd + 4 * (2k + hh)
  const int Tw = (T - hh + 1) >> 1;  // tail chains of this wave (0 or 1): segment nmain + hh
  const int nph = Mw > 0 ? Mw : Tw;

  // The segments phase 0 of any wave reads: its first main segment (simd + 4h), and the
  // tail as well where that phase is the wave's last.
  int s0 = -1;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int mw = (M - h + 1) >> 1;
    const int tw = (T - h + 1) >> 1;
    if (mw > 0) s0 = max(s0, min(3 + 4 * h, nmain - 1));
    if (mw <= 1 && tw > 0) s0 = max(s0, nmain + h);
  }
  const int rows0 = min(HR, fdiv(16 * s0 + 15 + a.vmax, a.fd_L) + 1);
  const int nblk = (HR * a.L + 15) >> 4;     // halo blocks per quad
  const int nblk0 = (rows0 * a.L + 15) >> 4;  // of which phase 0 reads the first nblk0

  // ---- every load, round-robin over the waves: instruction f goes to wave f % 8 ----
  constexpr int kFilt = 4 * KB;
  constexpr int kEp = EPI != kEpiAcc32 ? 2 : 0;
  int my = 0, my0 = 0;
  {
    const size_t img = static_cast<size_t>(n) * a.H * a.W * a.C + static_cast<size_t>(gi) * a.Cg;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + img, a.H * a.W * a.C - gi * a.Cg);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(gi) * a.Kg * a.Kdim, a.Kg * a.Kdim);
    const int hi0 = ho0 - a.ph;
    // halo block kb of quad q: lane (li, lg) reads virtual pixel 16*kb + li, chunk 4q + lg
    auto halo_load = [&](int q, int kb) {
      const int u = 16 * kb + li;
      const int row = fdiv(u, a.fd_L);
      const int col = u - row * a.L;
      const int hi = hi0 + row;
      const int wi = col - a.pw;
      const bool ok = row < HR && static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) &&
                      static_cast<unsigned>(wi) < static_cast<unsigned>(a.W);
      const unsigned voff = ok ? static_cast<unsigned>((hi * a.W + wi) * a.C + 64 * q + 16 * lg) : 0x40000000u;
      load_lds16(rx, halo + (q * a.qblocks + kb) * 64, voff, 0);
    };
    // halo blocks [kb0, kb1) of every quad: block kb of quad q goes to wave (kb - q) % 8
    auto halo_range = [&](int kb0, int kb1) {
      for (int q = 0; q < a.NQ; ++q) {
        for (int kb = kb0 + ((wave + q - kb0) & (kFlatWaves - 1)); kb < kb1; kb += kFlatWaves) {
          halo_load(q, kb);
          ++my;
        }
      }
    };
    halo_range(0, nblk0);
    // the filter: instruction u to wave u % 8
    for (int u = wave; u < kFilt; u += kFlatWaves) {
      if constexpr (KB & 1) {
        // contiguous: instruction u = kilobyte u of the tile's 64 rows; channels 32..63
        // (kilobytes 2KB and up) land 2 slots further on
        load_lds16(rw, filt + u * 64 + (u >= 2 * KB ? 2 : 0), 16u * lane, static_cast<unsigned>(k0 * a.Kdim + 1024 * u));
      } else {
        // fragment order: instruction u = (b, j) = (u / 4, u % 4)
        const unsigned lane_row = static_cast<unsigned>((16 * (li >> 2) + (li & 3)) * a.Kdim + 16 * lg);
        load_lds16(rw, filt + u * 64, lane_row, static_cast<unsigned>((k0 + 4 * (u & 3)) * a.Kdim + 64 * (u >> 2)));
      }
      ++my;
    }
    // bias (wave 6) and scales (wave 7) of the tile's 64 channels: lanes 0..15
    if constexpr (kEp > 0) {
      const size_t off = static_cast<size_t>(gi) * a.Kg + k0;
      if (wave == kFlatWaves - 2) {
        load_lds16(make_rsrc(a.bias ? a.bias + off : nullptr, a.bias ? 256 : 0), ep, 16u * lane, 0);
        ++my;
      } else if (wave == kFlatWaves - 1) {
        load_lds16(make_rsrc(a.wscale + off, 256), ep + 64, 16u * lane, 0);
        ++my;
      }
    }
    my0 = my;
    halo_range(nblk0, nblk);
  }
  wait_vmcnt63(my - my0);
  barrier_only();
  // the requantization multipliers act_scale * w_scale of the tile's 64 channels replace the
  // scales in LDS (read only after the second barrier, which publishes them)
  if constexpr (EPI != kEpiAcc32) {
    if (wave == 0) {
      float* sc = reinterpret_cast<float*>(ep + 64);
      sc[lane] = requant_multiplier(a.act_scale, sc[lane]);
    }
  }

  // ---- the filter in registers: A[b][j], lane (li, lg): channel 16*(li/4) + 4j + li%4,
  // bytes [64b + 16lg, +16) of its KRSC row; read from LDS in phase 0, in K-block order and
  // behind that phase's first fragments, so its matrix instructions start as they land ----
  v4i A[KB][4];
  auto load_A = [&](int b) {
    if constexpr (KB & 1) {
      const v4i* fb = filt + 4 * KB * (16 * (li >> 2) + (li & 3)) + lg + ((li >> 3) ? 2 : 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) A[b][j] = fb[16 * KB * j + 4 * b];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) A[b][j] = filt[(4 * b + j) * 64 + lane];
    }
  };
  // requantization multipliers of channels 16lg + 4j .. + 3, from LDS where a value group
  // starts (no registers hold them between phases)
  const unsigned ep_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(ep) & 0xffffffffu);
  auto mult_of = [&](int j) -> v4f {
    return *reinterpret_cast<const __attribute__((address_space(3))) v4f*>(
        static_cast<uintptr_t>(ep_addr + 1024u + 64u * lg + 16u * j));
  };
  // per-lane LDS byte address of its B fragment in segment 0, per K-block
  const unsigned halo_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(halo) & 0xffffffffu);
  unsigned baddr[KB];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    const int u = li + (a.tap[b] & 0xffffff);
    const int q = a.tap[b] >> 24;
    baddr[b] = halo_addr + 16u * static_cast<unsigned>((q * a.qblocks + (u >> 4)) * 64 + 16 * lg + (u & 15));
  }
  // the tail chain's A fragment (channel block `simd`): LDS byte address per K-block
  const unsigned filt_addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(filt) & 0xffffffffu);
  unsigned ta0;
  if constexpr (KB & 1) {
    ta0 = filt_addr + 16u * static_cast<unsigned>(4 * KB * (16 * (li >> 2) + 4 * simd + (li & 3)) + lg +
                                                  ((li >> 3) ? 2 : 0));
  } else {
    ta0 = filt_addr + 16u * static_cast<unsigned>(simd * 64 + lane);
  }
  auto ta_addr = [&](int b) -> unsigned { return (KB & 1) ? ta0 + 64u * b : ta0 + 4096u * b; };

  // ---- output: a buffer resource over the band's rows (image n, channels gi*Kg + k0 on) ----
  constexpr int kOB = EPI == kEpiI8 ? 1 : 4;
  const size_t out0 = (static_cast<size_t>(n) * a.Ho + ho0) * a.Wo * a.K + static_cast<size_t>(gi) * a.Kg + k0;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(static_cast<char*>(a.y) + out0 * kOB, bh * a.Wo * a.K * kOB);
  // lane's output byte offset for segment seg (2^30 more where the virtual pixel is dropped)
  auto out_off = [&](int seg, int chan) -> unsigned {
    const int v = 16 * seg + li;
    const int t = fdiv(v, a.fd_L);
    const int c = v - t * a.L;
    const bool ok = v < P && c < a.Wo;
    return static_cast<unsigned>(((t * a.Wo + c) * a.K + chan) * kOB) + (ok ? 0u : 0x40000000u);
  };
  constexpr float lo = RELU ? 0.0f : -128.0f;

  // one output value (j, r) of a 16-channel accumulator set: packing state in pk / u4
  auto epi_value = [&](const v4i (&acc)[4], int j, int r, const v4f& mj, v4i& pk, unsigned (&u4)[4], unsigned off) {
    if constexpr (EPI == kEpiI8) {
      u4[r] = __float_as_uint(requant_magic(acc[j][r], mj[r], lo));
      if (r == 3)
        pk[j] = static_cast<int>(pack4_magic(__uint_as_float(u4[0]), __uint_as_float(u4[1]), __uint_as_float(u4[2]),
                                             __uint_as_float(u4[3])));
      if (j == 3 && r == 3) {
        __builtin_amdgcn_raw_buffer_store_b128(pk, ry, off, 0, kStoreAux);
        store_gap(pk);
      }
    } else if constexpr (EPI == kEpiAcc32) {
      if (r == 3) {
        __builtin_amdgcn_raw_buffer_store_b128(acc[j], ry, off + 16u * j, 0, kStoreAux);
        store_gap(acc[j]);
      }
    } else {
      float v = static_cast<float>(acc[j][r]) * mj[r];
      if constexpr (RELU) v = (v > 0.0f) ? v : 0.0f;  // NaN and -0 -> +0
      u4[r] = __float_as_uint(v);
      if (r == 3) {
        const v4i pj = v4i{static_cast<int>(u4[0]), static_cast<int>(u4[1]), static_cast<int>(u4[2]),
                           static_cast<int>(u4[3])};
        __builtin_amdgcn_raw_buffer_store_b128(pj, ry, off + 16u * j, 0, kStoreAux);
        store_gap(pj);
      }
    }
  };
  // the tail chain's 4 values (channels 16lg + 4*simd + r) and their store
  auto tail_epilogue = [&](const v4i& tacc, unsigned off) {
    if constexpr (EPI == kEpiI8) {
      const v4f m = mult_of(simd);
      float c[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) c[r] = requant_magic(tacc[r], m[r], lo);
      const unsigned u = pack4_magic(c[0], c[1], c[2], c[3]);
      __builtin_amdgcn_raw_buffer_store_b32(static_cast<int>(u), ry, off, 0, kStoreAux);
      asm volatile("s_nop 1" : : "v"(u) : "memory");
    } else if constexpr (EPI == kEpiAcc32) {
      __builtin_amdgcn_raw_buffer_store_b128(tacc, ry, off, 0, kStoreAux);
      store_gap(tacc);
    } else {
      const v4f m = mult_of(simd);
      v4i f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = static_cast<float>(tacc[r]) * m[r];
        if constexpr (RELU) v = (v > 0.0f) ? v : 0.0f;
        f[r] = __float_as_int(v);
      }
      __builtin_amdgcn_raw_buffer_store_b128(f, ry, off, 0, kStoreAux);
      store_gap(f);
    }
  };

  v4i acc[4];       // the current phase's main segment
  v4i prev[4];      // the previous phase's, whose epilogue runs during this phase
  v4i tacc = v4i{0, 0, 0, 0};
  unsigned prev_off = 0;

  // One phase: the matrix instructions of the main segment `seg` (MAIN) and of the tail
  // chain on segment tseg (TAIL), with the epilogue of the previous phase's segment (PREV)
  // spread between them.  FIRST: phase 0, which also reads the filter into registers and
  // ends with the wait for the rest of the halo.
  auto phase = [&](auto main_t, auto tail_t, auto prev_t, auto first_t, int seg, int tseg) {
    constexpr bool MAIN = decltype(main_t)::value;
    constexpr bool TAIL = decltype(tail_t)::value;
    constexpr bool PREV = decltype(prev_t)::value;
    constexpr bool FIRST = decltype(first_t)::value;
    const unsigned sb = 1024u * static_cast<unsigned>(seg);
    const unsigned tb = 1024u * static_cast<unsigned>(tseg);
    // accumulators start at the bias of the lane's channels
    v4i bj[4];
    v4i tbias = v4i{0, 0, 0, 0};
    if constexpr (EPI != kEpiAcc32) {
      if constexpr (MAIN) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bj[j] = ep[4 * lg + j];
      }
      if constexpr (TAIL) tbias = ep[4 * lg + simd];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) bj[j] = v4i{0, 0, 0, 0};
    }
    constexpr int RS = KB < 2 ? KB : 2;  // B fragments read RS K-blocks ahead
    v4i B[RS], TB[RS], TA[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) {
      if constexpr (MAIN) B[r] = lds_read16(baddr[r] + sb);
      if constexpr (TAIL) {
        TB[r] = lds_read16(baddr[r] + tb);
        TA[r] = lds_read16(ta_addr(r));
      }
    }
    if constexpr (FIRST && MAIN) {
#pragma unroll
      for (int b = 0; b < KB; ++b) load_A(b);
    }
    __builtin_amdgcn_sched_barrier(0);
    // The previous segment's 16 values are spread over K-blocks E0 .. KB-1: a value's
    // conversion reads an accumulator of the previous phase, which is complete once this
    // phase's first K-blocks are issued behind it.  A value group's multipliers are read one
    // K-block before the group starts when KB >= 4 (at most one group starts per K-block),
    // else where it starts.
    constexpr int E0 = KB >= 4 ? 2 : 0;
    constexpr int NE = KB - E0;
    v4i pk = v4i{0, 0, 0, 0};
    unsigned u4[4] = {0u, 0u, 0u, 0u};
    v4f mj = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    v4f mn = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      if constexpr (MAIN) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b % RS], b == 0 ? bj[j] : acc[j], 0, 0, 0);
      }
      if constexpr (TAIL) tacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(TA[b % RS], TB[b % RS], b == 0 ? tbias : tacc, 0, 0, 0);
      if (b + RS < KB) {
        if constexpr (MAIN) B[b % RS] = lds_read16(baddr[b + RS] + sb);
        if constexpr (TAIL) {
          TB[b % RS] = lds_read16(baddr[b + RS] + tb);
          TA[b % RS] = lds_read16(ta_addr(b + RS));
        }
      }
      if constexpr (PREV) {
        const int e = b - E0;  // this K-block's share of the values: [16e/NE, 16(e+1)/NE)
        if (e >= 0) {
          const int v0 = (16 * e) / NE, v1 = (16 * (e + 1)) / NE;
#pragma unroll
          for (int v = v0; v < v1; ++v) {
            if ((v & 3) == 0) {
              if constexpr (KB >= 4) {
                mj = mn;
              } else if constexpr (EPI != kEpiAcc32) {
                mj = mult_of(v >> 2);
              }
            }
            epi_value(prev, v >> 2, v & 3, mj, pk, u4, prev_off);
          }
        }
        if constexpr (KB >= 4 && EPI != kEpiAcc32) {
          // the value group that starts in the next K-block, if one does
          const int en = e + 1;
          if (en >= 0 && en < NE) {
            const int w0 = (16 * en) / NE, w1 = (16 * (en + 1)) / NE;
#pragma unroll
            for (int v = w0; v < w1; ++v)
              if ((v & 3) == 0) mn = mult_of(v >> 2);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FIRST) {
      wait_vmcnt63(0);
      barrier_only();
    }
  };
  auto final_epilogue = [&](auto main_t, auto tail_t, int seg, int tseg) {
    constexpr bool MAIN = decltype(main_t)::value;
    constexpr bool TAIL = decltype(tail_t)::value;
    if constexpr (MAIN) {
      v4i pk = v4i{0, 0, 0, 0};
      unsigned u4[4] = {0u, 0u, 0u, 0u};
      const unsigned off = out_off(seg, 16 * lg);
      v4f m4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) m4[j] = EPI != kEpiAcc32 ? mult_of(j) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int v = 0; v < 16; ++v) epi_value(acc, v >> 2, v & 3, m4[v >> 2], pk, u4, off);
    }
    if constexpr (TAIL) tail_epilogue(tacc, out_off(tseg, 16 * lg + 4 * simd));
  };

  using F = std::false_type;
  using Tr = std::true_type;
  const int tseg = nmain + hh;  // this wave's tail segment (when Tw == 1)
  if (nph == 0) {
    wait_vmcnt63(0);
    barrier_only();
  } else if (Mw == 0) {
    // tail chain only (tiny bands): one phase
    phase(F{}, Tr{}, F{}, Tr{}, 0, tseg);
    final_epilogue(F{}, Tr{}, 0, tseg);
  } else {
    int seg = simd + 4 * hh;
    if (Mw == 1) {
      if (Tw) {
        phase(Tr{}, Tr{}, F{}, Tr{}, seg, tseg);
        final_epilogue(Tr{}, Tr{}, seg, tseg);
      } else {
        phase(Tr{}, F{}, F{}, Tr{}, seg, 0);
        final_epilogue(Tr{}, F{}, seg, 0);
      }
    } else {
      phase(Tr{}, F{}, F{}, Tr{}, seg, 0);
      for (int k = 1; k < Mw; ++k) {
#pragma unroll
        for (int j = 0; j < 4; ++j) prev[j] = acc[j];
        prev_off = out_off(seg, 16 * lg);
        seg += 8;
        if (k + 1 < Mw || !Tw) {
          phase(Tr{}, F{}, Tr{}, F{}, seg, 0);
        } else {
          phase(Tr{}, Tr{}, Tr{}, F{}, seg, tseg);
        }
      }
      if (Tw) {
        final_epilogue(Tr{}, Tr{}, seg, tseg);
      } else {
        final_epilogue(Tr{}, F{}, seg, 0);
      }
    }
  }
}

struct FlatPlan {
  int KB, NQ, L, rext, vmax, BH, bands_per_img, ktpg, qblocks;
  int filt_lds, ep_lds, halo_lds;
  size_t lds_bytes;
};

int flat_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Matrix instructions one SIMD issues for a band of bh rows (the busiest SIMD: main
// segments plus one tail chain).
long long flat_simd_mfma(int bh, int L, int Wo, int KB) {
  const long long P = static_cast<long long>(bh - 1) * L + Wo;
  const long long nseg = (P + 15) / 16;
  long long M = nseg / 4, T = nseg % 4;
  if (T == 3) {
    ++M;
    T = 0;
  }
  return M * 4 * KB + (T > 0 ? KB : 0);
}

bool flat_plan(const Geom& g, FlatPlan* p, std::string* why) {
  auto no = [&](const char* m) { if (why) *why = m; return false; };
  if (g.Cg % 64 != 0 || g.Cg == 0) return no("flat kernel needs (c/groups) % 64 == 0");
  if (g.Kg <= 0 || g.Kg % 64 != 0) return no("flat kernel needs (k/groups) % 64 == 0");
  if (g.sh != 1 || g.sw != 1) return no("flat kernel needs stride 1");
  if (g.dh < 1 || g.dw < 1 || g.ph < 0 || g.pw < 0) return no("flat kernel needs positive dilation and padding >= 0");
  if (g.R < 1 || g.S < 1) return no("flat kernel needs a non-empty filter");
  const long long kb = static_cast<long long>(g.R) * g.S * (g.Cg / 64);
  if (kb > kFlatMaxKB) return no("flat kernel filter does not fit in registers (R*S*c/groups > 576)");
  if (static_cast<long long>(g.H) * g.W * g.C >= (1LL << 30)) return no("flat kernel needs images below 2^30 bytes");
  if (static_cast<long long>(g.Kg) * g.R * g.S * g.Cg >= (1LL << 30)) return no("flat kernel needs group filters below 2^30 bytes");
  if (static_cast<long long>(g.Ho) * g.Wo * g.K * 4 >= (1LL << 30)) return no("flat kernel needs images below 2^30 output bytes");
  const long long L = static_cast<long long>(g.Wo) + static_cast<long long>(g.S - 1) * g.dw;
  const long long rext = static_cast<long long>(g.R - 1) * g.dh;
  const long long vmax = rext * L + static_cast<long long>(g.S - 1) * g.dw;
  if (L > 4096 || vmax >= (1 << 20)) return no("flat kernel needs a narrow halo");
  p->KB = static_cast<int>(kb);
  p->NQ = g.Cg / 64;
  p->L = static_cast<int>(L);
  p->rext = static_cast<int>(rext);
  p->vmax = static_cast<int>(vmax);
  p->ktpg = g.Kg / 64;
  const int cus = flat_cu_count();
  const size_t filt_bytes = static_cast<size_t>(flat_filter_bytes(p->KB));
  bool found = false;
  double best = 0.0;
  for (int bh = 1; bh <= g.Ho; ++bh) {
    const long long HR = bh + rext;
    // blocks of the halo read: up to the last segment's pixels plus the largest shift
    const long long nseg = ((bh - 1) * L + g.Wo + 15) / 16 + 4;  // a junk main segment at most
    const long long qblocks = std::max((HR * L + 15) / 16, (16 * nseg + vmax + 15) / 16);
    const size_t lds = filt_bytes + 2048 + static_cast<size_t>(p->NQ * qblocks) * 1024;
    if (lds > static_cast<size_t>(kFlatLds)) break;
    const long long loads = p->NQ * ((HR * L + 15) / 16) + 4 * p->KB + 2;
    if (loads > 63LL * kFlatWaves) break;  // vmcnt counts 63 loads per wave
    const long long bands = (g.Ho + bh - 1) / bh;
    const long long wgs = static_cast<long long>(g.N) * bands * g.G * p->ktpg;
    const long long rounds = (wgs + cus - 1) / cus;
    // cycles of one round: matrix instructions at ~75% of 16 clocks (with the epilogue
    // spread among them) plus start-up (launch, first loads) and the loads of the band
    const double mfma = static_cast<double>(flat_simd_mfma(bh, static_cast<int>(L), g.Wo, p->KB)) * 16.0 / 0.75;
    const double load = 2400.0 + static_cast<double>(filt_bytes + p->NQ * HR * L * 64) / 40.0;
    const double cost = static_cast<double>(rounds) * (mfma + load);
    if (!found || cost < best - 1e-9) {
      found = true;
      best = cost;
      p->BH = bh;
      p->bands_per_img = static_cast<int>(bands);
      p->qblocks = static_cast<int>(qblocks);
      p->filt_lds = 0;
      p->ep_lds = static_cast<int>(filt_bytes);
      p->halo_lds = static_cast<int>(filt_bytes + 2048);
      p->lds_bytes = lds;
    }
  }
  if (!found) return no("flat kernel halo does not fit in LDS");
  const long long blocks = static_cast<long long>(g.N) * p->bands_per_img * g.G * p->ktpg;
  if (blocks > 0x7fffffffLL) return no("grid too large");
  return true;
}

template <int KB>
void flat_launch_kb(const FlatArgs& a, const FlatPlan& pl, Epi epi, unsigned nblocks, hipStream_t stream) {
  const dim3 grid(nblocks);
  auto go = [&](auto kern) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(pl.lds_bytes));
    hipLaunchKernelGGL(kern, grid, dim3(64 * kFlatWaves), pl.lds_bytes, stream, a);
  };
  switch (epi) {
    case kEpiI8: a.relu ? go(i8_flat_kernel<KB, kEpiI8, true>) : go(i8_flat_kernel<KB, kEpiI8, false>); break;
    case kEpiAcc32: go(i8_flat_kernel<KB, kEpiAcc32, false>); break;
    default: a.relu ? go(i8_flat_kernel<KB, kEpiF32, true>) : go(i8_flat_kernel<KB, kEpiF32, false>); break;
  }
}

template <int KB>
void flat_dispatch(int kb, const FlatArgs& a, const FlatPlan& pl, Epi epi, unsigned nblocks, hipStream_t stream) {
  if constexpr (KB >= 1) {
    if (kb == KB) {
      flat_launch_kb<KB>(a, pl, epi, nblocks, stream);
    } else {
      flat_dispatch<KB - 1>(kb, a, pl, epi, nblocks, stream);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool flat_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                   std::string* why) {
  const bool params_ok = epi == kEpiAcc32 || ((rq.bias == nullptr || aligned16(rq.bias)) && aligned16(rq.wscale));
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || !params_ok) {
    if (why) *why = "flat kernel needs 16-byte aligned tensors, bias and scales";
    return false;
  }
  FlatPlan pl;
  return flat_plan(g, &pl, why);
}

hipError_t launch_i8_flat(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  FlatPlan pl;
  if (!flat_plan(g, &pl, nullptr)) return hipErrorInvalidConfiguration;
  FlatArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw;
  a.Cg = g.Cg; a.Kg = g.Kg; a.Kdim = g.R * g.S * g.Cg;
  a.L = pl.L; a.rext = pl.rext; a.vmax = pl.vmax;
  a.BH = pl.BH; a.bands_per_img = pl.bands_per_img; a.ktpg = pl.ktpg;
  a.ntiles = g.G * pl.ktpg;
  a.NQ = pl.NQ; a.qblocks = pl.qblocks;
  a.filt_lds = pl.filt_lds; a.ep_lds = pl.ep_lds; a.halo_lds = pl.halo_lds;
  a.act_scale = rq.act_scale; a.relu = rq.relu;
  // K-block b = 64 consecutive reduction bytes: tap b / NQ, quad b % NQ
  for (int b = 0; b < kFlatMaxKB; ++b) {
    if (b < pl.KB) {
      const int tap = b / pl.NQ;
      const int q = b % pl.NQ;
      const int r = tap / g.S;
      const int s = tap % g.S;
      a.tap[b] = q << 24 | (r * g.dh * pl.L + s * g.dw);
    } else {
      a.tap[b] = 0;
    }
  }
  a.fd_ntiles = fastdiv_m(a.ntiles);
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_ktpg = fastdiv_m(pl.ktpg);
  a.fd_L = fastdiv_m(pl.L);
  const long long nblocks = static_cast<long long>(g.N) * pl.bands_per_img * a.ntiles;
  a.nblocks = static_cast<int>(nblocks);
  flat_dispatch<kFlatMaxKB>(pl.KB, a, pl, epi, static_cast<unsigned>(nblocks), stream);
  return hipGetLastError();
}

}  // namespace miq
