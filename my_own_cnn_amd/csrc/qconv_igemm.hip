// int8 implicit-GEMM convolution on the gfx950 matrix cores (v_mfma_i32_16x16x64_i8).
//
// GEMM view: rows = output channels (A operand = KRSC filter), columns = output pixels
// (B operand = NHWC input patches), reduction = (r, s, ci).  The reduction runs over
// "chunks" of 16 consecutive input channels of one tap (q = tap * Cg/16 + ci/16); one
// MFMA K-block holds 4 chunks, lane group g = lane/16 feeding chunk 4b+g with 16 bytes.
// A and B use the same lane <-> chunk assignment, so the hardware's internal byte order
// inside a K-block does not matter.
//
// Output-channel permutation: MFMA j (0..3) of a 64-channel tile maps its row rho to
// channel 16*(rho/4) + 4*j + rho%4.  Each lane then ends up holding 16 consecutive
// channels of one pixel (4 rows x 4 MFMAs), which the epilogue writes as one 16-byte
// int8 store (or four 16-byte int32/fp32 stores): a wave writes 16 pixels x 64 channels.
//
// Work decomposition: a workgroup (WAVES = 4 or 8 waves) owns one tile of RB output rows x
// CB output columns of one image (one pass of every wave: at most WAVES_P*NSEG 16-pixel
// segments, interleaved over the waves) and KT_WG = 64*NKT*WAVES_K output channels of one
// group.  Each wave computes NKT 64-channel tiles x up to NSEG segments; per K-block it
// reads 4*NKT filter fragments and one input fragment per segment (1 KB each) from LDS.
// The host picks the tile so that every SIMD gets as even a share of segments as the
// problem allows (8-wave workgroups let one filter copy in LDS serve a whole CU).
//
// LDS holds, per workgroup: the bias and requantization multiplier of its channels; the
// filter, in fragment order (one 1 KB block per (K-block, 64-channel tile, j), lane l's 16
// bytes at l*16), staged in chunks of K-blocks; and the input patch of the tile (its
// "halo": rows*stride + dilated taps, all Cg channels, zero where the convolution pads),
// stored planar as [chunk c16][column parity hc % sw][row][hc / sw] x 16 bytes.  In that
// layout the 16 lanes of an MFMA lane group, which read one chunk of 16 consecutive output
// pixels, read 256 contiguous bytes for any stride: no bank conflicts, and the address of
// a fragment is a per-lane constant plus a per-K-block constant.  Every runtime division
// is a multiply-high by a host-computed magic number.  Filter and halo arrive with direct global->LDS loads
// (global_load_lds_dwordx4): no registers, all in flight at once.  When the filter does
// not fit, the chunk after the current one streams in while the current one computes.
//
// The K-loop is software-pipelined: the fragments of K-block b+1 are read from LDS while
// the MFMAs of K-block b run.  Accumulators start at the bias, so the epilogue is
// convert, scale, clamp, round: round-to-nearest-even comes from adding 1.5*2^23 to the
// clamped value (exact IEEE rounding of a value in [-128, 127]: the sum lands in
// [2^23, 2^24), where the float grid is the integers), whose low byte is then the
// two's-complement int8 result.

#include "qconv_device.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace miq {
namespace {

constexpr int kLdsBudget = 160 * 1024;   // LDS bytes per workgroup on gfx950
constexpr int kLdsPreferred = 76 * 1024; // two workgroups per CU

struct IgemmArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  void* y;
  int H, W, C, K, R, S, Ho, Wo;
  int ph, pw, sh, sw, dh, dw;
  int Cg, Kg, Cg16;  // channels per group, output channels per group, Cg / 16
  int NQ, KB, Kdim;  // chunks per filter row, MFMA K-blocks, R*S*Cg
  int KBC, nchunks;  // K-blocks per staged filter chunk, number of chunks
  int RB, CB;        // output tile extent
  int tiles_h, tiles_w;
  int kt_per_group;  // channel tiles (of KT_WG) per group
  int HCs, PS, nslot;  // halo: columns per parity plane, plane size and total size (16-byte slots)
  int w_off, h_off;  // LDS byte offsets of the filter buffers and of the halo
  int w_buf_bytes;   // bytes of one filter chunk buffer
  float act_scale;
  int relu;
  FastDiv fd_ps, fd_hcs, fd_sw, fd_cb, fd_cg16, fd_s, fd_tiles_img, fd_tiles_w, fd_ktpg, fd_gx;
};

// Workgroups are dispatched round-robin over the 8 XCDs (id % 8).  Give each XCD a
// contiguous range of tile ids so neighbouring tiles, which share halo rows, meet in the
// same L2.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
  const int q = total >> 3;
  const int r = total & 7;
  const int xcd = bid & 7;
  const int pos = bid >> 3;
  return xcd * q + min(xcd, r) + pos;
}

// 16 bytes global -> LDS without registers; `lds_wave_base` is the wave's 1 KB block, lane l
// lands at lds_wave_base + 16*l.
__device__ __forceinline__ void load_lds16(const void* src, v4i* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
}

// Filter fragments of K-blocks [b0, b0 + nb) of the workgroup's channels into `dst`
// (fragment order).  Fragment f = (bl * CT + ct) * 4 + j goes to dst + f * 64 (v4i units).
template <int CT, int WAVES>
__device__ __forceinline__ void stage_filter(const IgemmArgs& a, const int8_t* wg, int kwg0, int b0, int nb, v4i* dst,
                                             int wave, int lane) {
  const int nfrag = nb * CT * 4;
  const int row_l = lane & 15;
  const int grp_l = lane >> 4;
  for (int f = wave; f < nfrag; f += WAVES) {
    const int j = f & 3;
    const int ct = (f >> 2) % CT;
    const int bl = (f >> 2) / CT;
    const int kc = kwg0 + ct * 64 + 16 * (row_l >> 2) + 4 * j + (row_l & 3);
    const int q = 4 * (b0 + bl) + grp_l;
    v4i* blk = dst + f * 64;
    if (kc < a.Kg && q < a.NQ) {
      load_lds16(wg + static_cast<size_t>(kc) * a.Kdim + q * 16, blk);
    } else {
      blk[lane] = v4i{0, 0, 0, 0};
    }
  }
}

// Scheduling groups for one K-block step: MFMA, LDS read, MFMA, LDS read, ... then the
// remaining MFMAs (or reads).
template <int NMFMA, int NREAD>
__device__ __forceinline__ void interleave_mfma_ds() {
  if constexpr (NMFMA > 0 && NREAD > 0) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
    interleave_mfma_ds<NMFMA - 1, NREAD - 1>();
  } else if constexpr (NMFMA > 0) {
    __builtin_amdgcn_sched_group_barrier(0x008, NMFMA, 0);
  } else if constexpr (NREAD > 0) {
    __builtin_amdgcn_sched_group_barrier(0x100, NREAD, 0);
  }
}

// Calls f(std::integral_constant<int, n>) for a wave-uniform 1 <= n <= NMAX (nothing for n
// == 0): one branch-free instantiation of the callee per count.
template <int NMAX, typename F>
__device__ __forceinline__ void dispatch_count(int n, F&& f) {
  if constexpr (NMAX > 0) {
    if (n == NMAX) {
      f(std::integral_constant<int, NMAX>{});
    } else {
      dispatch_count<NMAX - 1>(n, f);
    }
  }
}

template <int NKT, int NSEG, int WAVES_K, int EPI, bool TAPU, int WAVES>
__global__ void __launch_bounds__(64 * WAVES, (NKT == 1 && WAVES == 4) ? 2 : 1)  // two waves per SIMD
i8_igemm_kernel(IgemmArgs a) {
  constexpr int WAVES_P = WAVES / WAVES_K;
  constexpr int KTILE = 64 * NKT;          // output channels per wave
  constexpr int KT_WG = KTILE * WAVES_K;   // output channels per workgroup
  constexpr int CT = KT_WG / 64;           // 64-channel tiles per workgroup
  extern __shared__ v4i smem[];
  int32_t* ep_bias = reinterpret_cast<int32_t*>(smem);
  float* ep_mult = reinterpret_cast<float*>(smem) + KT_WG;
  v4i* wbuf0 = smem + a.w_off / 16;
  v4i* wbuf1 = wbuf0 + a.w_buf_bytes / 16;
  v4i* halo = smem + a.h_off / 16;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: wave-level branches stay scalar
  const int wk = wave % WAVES_K;
  const int wp = wave / WAVES_K;
  const int row_l = lane & 15;  // MFMA row (A) / column (B) of this lane
  const int grp_l = lane >> 4;  // chunk slot of this lane inside a K-block

  const int nblk = gridDim.x * gridDim.y;
  const int lin = xcd_tile(blockIdx.x + blockIdx.y * gridDim.x, nblk);
  const int ctile = fdiv(lin, a.fd_gx);
  const int tile = lin - ctile * static_cast<int>(gridDim.x);
  const int n = fdiv(tile, a.fd_tiles_img);
  const int trem = tile - n * a.tiles_h * a.tiles_w;
  const int th = fdiv(trem, a.fd_tiles_w);
  const int tw = trem - th * a.tiles_w;
  const int gi = fdiv(ctile, a.fd_ktpg);
  const int kt = ctile - gi * a.kt_per_group;
  const int kwg0 = kt * KT_WG;             // first channel of the workgroup within the group
  const int kwave0 = kwg0 + wk * KTILE;    // first channel of this wave within the group
  const int8_t* wg = a.w + static_cast<size_t>(gi) * a.Kg * a.Kdim;

  const int ho0 = th * a.RB;
  const int wo0 = tw * a.CB;
  const int rows = min(a.RB, a.Ho - ho0);
  const int cols = min(a.CB, a.Wo - wo0);

  // ---- staging: filter chunk 0 and the halo (direct loads), epilogue parameters ----
  stage_filter<CT, WAVES>(a, wg, kwg0, 0, min(a.KBC, a.KB), wbuf0, wave, lane);
  {
    const int hi0 = ho0 * a.sh - a.ph;
    const int wi0 = wo0 * a.sw - a.pw;
    const int8_t* xg = a.x + static_cast<size_t>(n) * a.H * a.W * a.C + static_cast<size_t>(gi) * a.Cg;
    for (int u = wave; u * 64 < a.nslot; u += WAVES) {
      const int L = u * 64 + lane;  // LDS slot this lane fills
      if (L < a.nslot) {
        const int plane = fdiv(L, a.fd_ps);
        const int rem = L - plane * a.PS;
        const int hr = fdiv(rem, a.fd_hcs);
        const int hcs = rem - hr * a.HCs;
        const int c16 = fdiv(plane, a.fd_sw);
        const int par = plane - c16 * a.sw;
        const int hi = hi0 + hr;
        const int wi = wi0 + hcs * a.sw + par;
        if (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) && static_cast<unsigned>(wi) < static_cast<unsigned>(a.W)) {
          load_lds16(xg + (static_cast<size_t>(hi) * a.W + wi) * a.C + c16 * 16, halo + u * 64);
        } else {
          halo[L] = v4i{0, 0, 0, 0};
        }
      }
    }
  }
  if constexpr (EPI != kEpiAcc32) {
    stage_requant<EPI>(Requant{a.bias, a.wscale, a.act_scale, a.relu}, gi * a.Kg + kwg0, a.Kg - kwg0, KT_WG, ep_bias,
                       ep_mult);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const bool wave_active = kwave0 < a.Kg;  // waves past the last channel still join every barrier

  // per segment: halo slot of tap (0,0) / chunk 0 for this lane's pixel, output pixel index.
  // Segments are interleaved over the waves: segment i of this wave is tile segment
  // wp + i * WAVES_P, and the first nsv of them exist (wave-uniform).
  const int nseg_tile = (rows * a.CB + 15) >> 4;
  const int nsv = wave_active ? min(NSEG, max(0, (nseg_tile - wp + WAVES_P - 1) / WAVES_P)) : 0;
  int pix_off[NSEG], opix[NSEG];
  bool pv[NSEG];
#pragma unroll
  for (int i = 0; i < NSEG; ++i) {
    const int p = (wp + i * WAVES_P) * 16 + row_l;
    const int lho = fdiv(p, a.fd_cb);
    const int lwo = p - lho * a.CB;
    pv[i] = lho < rows && lwo < cols;
    // pixels outside the tile read slot 0 (finite data, never stored): no predication in the K-loop
    pix_off[i] = pv[i] ? lho * a.sh * a.HCs + lwo : 0;
    opix[i] = (n * a.Ho + ho0 + lho) * a.Wo + wo0 + lwo;
  }
  const int grp_plane_off = grp_l * a.sw * a.PS;  // lane group g reads chunk c16 + g (TAPU)

  // accumulators start at the bias (int8 / fp32 outputs) or at 0 (raw accumulators)
  v4i acc[NKT][4][NSEG];
#pragma unroll
  for (int t = 0; t < NKT; ++t) {
    const int lc = wk * KTILE + t * 64 + 16 * grp_l;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v4i init = {0, 0, 0, 0};
      if constexpr (EPI != kEpiAcc32) init = reinterpret_cast<const v4i*>(ep_bias + lc)[j];
#pragma unroll
      for (int i = 0; i < NSEG; ++i) acc[t][j][i] = init;
    }
  }

  // fragment loaders for one K-block; `b` is clamped by the callers to [0, KB)
  auto load_b = [&](int b, auto& B) {
    constexpr int NS = std::extent<std::remove_reference_t<decltype(B)>>::value;
    int off;
    if constexpr (TAPU) {  // Cg16 % 4 == 0: the 4 chunks of a K-block belong to one tap
      const int q0 = 4 * b;
      const int tap = fdiv(q0, a.fd_cg16);
      const int cb = q0 - tap * a.Cg16;
      const int rr = fdiv(tap, a.fd_s);
      const int sdw = (tap - rr * a.S) * a.dw;
      const int hq = fdiv(sdw, a.fd_sw);
      off = (cb * a.sw + (sdw - hq * a.sw)) * a.PS + rr * a.dh * a.HCs + hq + grp_plane_off;
    } else {
      const int q = min(4 * b + grp_l, a.NQ - 1);  // past the last chunk the filter fragment is zero
      const int tap = fdiv(q, a.fd_cg16);
      const int c16 = q - tap * a.Cg16;
      const int rr = fdiv(tap, a.fd_s);
      const int sdw = (tap - rr * a.S) * a.dw;
      const int hq = fdiv(sdw, a.fd_sw);
      off = (c16 * a.sw + (sdw - hq * a.sw)) * a.PS + rr * a.dh * a.HCs + hq;
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) B[i] = halo[pix_off[i] + off];
  };
  auto load_a = [&](const v4i* wb, int bl, v4i (&A)[NKT][4]) {
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) A[t][j] = wb[((bl * CT + wk * NKT + t) * 4 + j) * 64 + lane];
  };
  auto mma = [&](const v4i (&A)[NKT][4], const auto& B) {
    constexpr int NS = std::extent<std::remove_reference_t<decltype(B)>>::value;
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[t][j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[t][j], B[i], acc[t][j][i], 0, 0, 0);
  };
  // K-blocks [b0, b0 + nb) of the staged chunk `wb` for the first NS segments; branch-free
  // inside, so LDS reads of K-block b+1 stay in flight under the MFMAs of K-block b.
  auto kloop = [&](auto ns_tag, const v4i* wb, int b0, int nb) {
    constexpr int NS = decltype(ns_tag)::value;
    v4i A0[NKT][4], A1[NKT][4], B0[NS], B1[NS];
    load_a(wb, 0, A0);
    load_b(b0, B0);
    int bl = 0;
    // The reads of the next K-block are interleaved one by one with the first MFMAs of
    // this one, so they complete under the remaining MFMAs.
    constexpr int NMMA = NKT * 4 * NS, NRD = NKT * 4 + NS;
    for (; bl + 2 <= nb; bl += 2) {
      mma(A0, B0);
      load_a(wb, bl + 1, A1);
      load_b(b0 + bl + 1, B1);
      interleave_mfma_ds<NMMA, NRD>();
      const int bn = min(bl + 2, nb - 1);  // the last pass re-reads a valid K-block, unused
      mma(A1, B1);
      load_a(wb, bn, A0);
      load_b(b0 + bn, B0);
      interleave_mfma_ds<NMMA, NRD>();
    }
    if (bl < nb) mma(A0, B0);
  };

  for (int c = 0; c < a.nchunks; ++c) {
    const int b0 = c * a.KBC;
    const int nb = min(a.KBC, a.KB - b0);
    const v4i* wb = (c & 1) ? wbuf1 : wbuf0;
    if (c + 1 < a.nchunks) {  // next chunk streams in behind this one
      stage_filter<CT, WAVES>(a, wg, kwg0, b0 + a.KBC, min(a.KBC, a.KB - b0 - a.KBC), (c & 1) ? wbuf0 : wbuf1, wave,
                               lane);
    }
    dispatch_count<NSEG>(nsv, [&](auto ns_tag) { kloop(ns_tag, wb, b0, nb); });
    if (c + 1 < a.nchunks) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  if (!wave_active) return;

  // ---- epilogue: lane holds channels kc0 .. kc0+15 of pixel p for each (t, i) ----
#pragma unroll
  for (int t = 0; t < NKT; ++t) {
    const int kc0 = kwave0 + t * 64 + 16 * grp_l;
    if (kc0 >= a.Kg) continue;
    const int kabs = gi * a.Kg + kc0;
    const bool full = (kc0 + 16 <= a.Kg) && ((a.Kg & 15) == 0);
    const int lc = kc0 - kwg0;
#pragma unroll
    for (int i = 0; i < NSEG; ++i) {
      if (!pv[i]) continue;
      store16_biased<EPI>(a.y, static_cast<size_t>(opix[i]) * a.K + kabs, acc[t][0][i], acc[t][1][i], acc[t][2][i],
                          acc[t][3][i], kc0, a.Kg, full, ep_mult + lc, a.relu);
    }
  }
}

// Host-side tiling decision for one problem.
struct IgemmPlan {
  int nkt, waves_k, nseg, waves;
  int KBC, nchunks;
  int RB, CB, tiles_h, tiles_w, kt_per_group;
  int w_off, h_off, w_buf_bytes;
  size_t lds_bytes;
};

// Planar halo of a full RB x CB tile: Cg16 chunks x sw parity planes x HR rows x HCs columns.
struct HaloDims {
  int HR, HCs, PS, nslot;
};

HaloDims halo_dims(const Geom& g, int RB, int CB) {
  HaloDims h;
  h.HR = (RB - 1) * g.sh + (g.R - 1) * g.dh + 1;
  const int HC = (CB - 1) * g.sw + (g.S - 1) * g.dw + 1;
  h.HCs = (HC + g.sw - 1) / g.sw;
  h.PS = h.HR * h.HCs;
  h.nslot = (g.Cg / 16) * g.sw * h.PS;
  return h;
}

size_t halo_bytes(const Geom& g, int RB, int CB) {
  const long long HR = static_cast<long long>(RB - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
  const long long HC = static_cast<long long>(CB - 1) * g.sw + static_cast<long long>(g.S - 1) * g.dw + 1;
  const long long HCs = (HC + g.sw - 1) / g.sw;
  return static_cast<size_t>(HR * HCs * g.sw * g.Cg);
}

size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Compute units of the current device (one query per device; 256 when no device answers).
int device_cu_count() {
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

// Chooses the channel split, the workgroup size (4 or 8 waves) and the tile.  The cost of a
// candidate is, per round of resident workgroups, the largest number of 16-pixel segments
// one SIMD works through, plus a share for the segments of the whole CU (LDS and L1
// bandwidth are per CU) and a fixed per-round cost for staging and the epilogue; the
// cheapest candidate wins (ties: taller tiles, which re-read less halo).
bool make_plan(const Geom& g, IgemmPlan* pl) {
  if (g.Kg <= 64) {
    pl->nkt = 1; pl->waves_k = 1;
  } else if (g.Kg <= 128) {
    pl->nkt = 1; pl->waves_k = 2;
  } else if (g.Kg <= 256) {
    pl->nkt = 1; pl->waves_k = 4;
  } else {
    pl->nkt = 2; pl->waves_k = 4;
  }
  pl->nseg = pl->nkt == 2 ? 2 : 4;  // keeps two waves per SIMD (registers)
  const int kt_wg = 64 * pl->nkt * pl->waves_k;
  pl->kt_per_group = (g.Kg + kt_wg - 1) / kt_wg;
  const int kb = (g.R * g.S * (g.Cg / 16) + 3) / 4;
  const size_t kblock_bytes = static_cast<size_t>(kt_wg) * 64;  // filter bytes of one K-block
  const size_t ep_bytes = round_up(static_cast<size_t>(kt_wg) * 8, 1024);
  const int cus = device_cu_count();
  auto lds_total = [&](int rb, int cb, int kbc, int nbuf) {
    return ep_bytes + nbuf * kbc * kblock_bytes + round_up(halo_bytes(g, rb, cb), 1024);
  };

  bool found = false;
  double best = 0.0;
  for (int waves : {4, 8}) {
    if (waves == 8 && pl->nkt != 1) continue;
    const int waves_p = waves / pl->waves_k;
    const int pass_segs = waves_p * pl->nseg;
    // Filter staging: whole when that keeps two workgroups per CU (4-wave) / fits (8-wave);
    // else the largest double-buffered chunk that does; else anything within the full LDS.
    const size_t preferred = waves == 4 ? 76 * 1024 : static_cast<size_t>(kLdsBudget);
    auto fit = [&](int rb, int cb, int* kbc, int* nbuf) {
      const size_t limits[2] = {preferred, static_cast<size_t>(kLdsBudget)};
      for (size_t lim : limits) {
        if (lds_total(rb, cb, kb, 1) <= lim) {
          *kbc = kb;
          *nbuf = 1;
          return true;
        }
        for (int c = kb - 1; c >= 1; --c) {
          if (lds_total(rb, cb, c, 2) <= lim) {
            *kbc = c;
            *nbuf = 2;
            return true;
          }
        }
      }
      return false;
    };
    int CB = std::min(g.Wo, pass_segs * 16);
    int kbc = 0, nbuf = 0;
    while (CB > 16 && !fit(1, CB, &kbc, &nbuf)) CB -= 16;
    if (!fit(1, CB, &kbc, &nbuf)) continue;
    const int tiles_w = (g.Wo + CB - 1) / CB;
    for (int rb = 1; rb <= g.Ho; ++rb) {
      const int segs = (rb * CB + 15) / 16;
      if (segs > pass_segs) break;
      if (!fit(rb, CB, &kbc, &nbuf)) break;
      const size_t lds = lds_total(rb, CB, kbc, nbuf);
      const long long tiles = static_cast<long long>(g.N) * ((g.Ho + rb - 1) / rb) * tiles_w * g.G * pl->kt_per_group;
      const int wg_per_cu = (waves == 8 || lds > 76 * 1024) ? 1 : 2;
      const long long rounds = (tiles + static_cast<long long>(cus) * wg_per_cu - 1) / (static_cast<long long>(cus) * wg_per_cu);
      // segments of the busiest SIMD in one round: SIMD s runs waves s, s+4 of the resident workgroups
      auto segs_of = [&](int wp) { return wp < segs % waves_p ? segs / waves_p + 1 : segs / waves_p; };
      int per_simd = 0;
      const int per_cu = (waves == 8 ? 1 : wg_per_cu) * segs;  // shares LDS / L1 bandwidth of one CU
      for (int sm = 0; sm < 4; ++sm) {
        int load = 0;
        if (waves == 8) {
          load = segs_of(sm / pl->waves_k) + segs_of((sm + 4) / pl->waves_k);
        } else {
          load = wg_per_cu * segs_of(sm / pl->waves_k);
        }
        per_simd = std::max(per_simd, load);
      }
      const double cost = static_cast<double>(rounds) * (per_simd + 0.125 * per_cu + 3.0 * wg_per_cu);
      if (!found || cost < best - 1e-9 || (cost <= best + 1e-9 && rb >= pl->RB && waves == pl->waves)) {
        found = true;
        best = cost;
        pl->waves = waves;
        pl->RB = rb;
        pl->CB = CB;
        pl->KBC = kbc;
        pl->nchunks = (kb + kbc - 1) / kbc;
        pl->tiles_h = (g.Ho + rb - 1) / rb;
        pl->tiles_w = tiles_w;
        pl->w_off = static_cast<int>(ep_bytes);
        pl->w_buf_bytes = static_cast<int>(kbc * kblock_bytes);
        pl->h_off = static_cast<int>(ep_bytes + nbuf * kbc * kblock_bytes);
        pl->lds_bytes = lds;
      }
    }
  }
  return found;
}

template <int NKT, int NSEG, int WAVES_K, int EPI, bool TAPU, int WAVES>
void launch_cfg(const IgemmArgs& a, const IgemmPlan& pl, int N, int G, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(N * pl.tiles_h * pl.tiles_w), static_cast<unsigned>(G * pl.kt_per_group));
  auto kern = i8_igemm_kernel<NKT, NSEG, WAVES_K, EPI, TAPU, WAVES>;
  if (pl.lds_bytes > 64 * 1024) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(pl.lds_bytes));
  }
  hipLaunchKernelGGL(kern, grid, dim3(64 * WAVES), pl.lds_bytes, stream, a);
}

template <int NKT, int WAVES_K, int EPI, bool TAPU>
void launch_nseg(const IgemmArgs& a, const IgemmPlan& pl, int N, int G, hipStream_t stream) {
  if constexpr (NKT == 2) {
    launch_cfg<NKT, 2, WAVES_K, EPI, TAPU, 4>(a, pl, N, G, stream);
  } else {
    if (pl.waves == 8) {
      launch_cfg<NKT, 4, WAVES_K, EPI, TAPU, 8>(a, pl, N, G, stream);
    } else {
      launch_cfg<NKT, 4, WAVES_K, EPI, TAPU, 4>(a, pl, N, G, stream);
    }
  }
}

template <int EPI, bool TAPU>
void launch_shape(const IgemmArgs& a, const IgemmPlan& pl, int N, int G, hipStream_t stream) {
  if (pl.nkt == 2) {
    launch_nseg<2, 4, EPI, TAPU>(a, pl, N, G, stream);
  } else if (pl.waves_k == 4) {
    launch_nseg<1, 4, EPI, TAPU>(a, pl, N, G, stream);
  } else if (pl.waves_k == 2) {
    launch_nseg<1, 2, EPI, TAPU>(a, pl, N, G, stream);
  } else {
    launch_nseg<1, 1, EPI, TAPU>(a, pl, N, G, stream);
  }
}

template <int EPI>
void launch_epi(const IgemmArgs& a, const IgemmPlan& pl, int N, int G, hipStream_t stream) {
  if (a.Cg16 % 4 == 0) {
    launch_shape<EPI, true>(a, pl, N, G, stream);
  } else {
    launch_shape<EPI, false>(a, pl, N, G, stream);
  }
}

// 1x1 / stride 1 / no padding: every output pixel reads exactly its own input pixel, so
// the batch is one long row and tiles need no halo.
Geom canonical(const Geom& g) {
  Geom c = g;
  if (g.R == 1 && g.S == 1 && g.sh == 1 && g.sw == 1 && g.ph == 0 && g.pw == 0 && g.Ho == g.H && g.Wo == g.W) {
    const long long pix = static_cast<long long>(g.N) * g.H * g.W;
    if (pix <= 0x7fffffffLL) {
      c.N = 1; c.H = 1; c.W = static_cast<int>(pix); c.Ho = 1; c.Wo = c.W;
    }
  }
  return c;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool igemm_eligible(const Geom& g0, const void* x, const void* w, const void* y, Epi epi, std::string* why) {
  (void)epi;
  const Geom g = canonical(g0);
  auto no = [&](const char* m) { if (why) *why = m; return false; };
  if (g.Cg % 16 != 0) return no("implicit GEMM needs (c/groups) % 16 == 0");
  if (g.Cg == 0 || g.Kg == 0) return no("implicit GEMM needs at least one channel per group");
  if (g.sh < 1 || g.sw < 1 || g.dh < 1 || g.dw < 1) return no("implicit GEMM needs stride and dilation >= 1");
  if (g.ph < 0 || g.pw < 0) return no("implicit GEMM needs non-negative padding");
  if (g.R < 1 || g.S < 1) return no("implicit GEMM needs a non-empty filter");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y)) return no("implicit GEMM needs 16-byte aligned tensors");
  IgemmPlan pl;
  if (!make_plan(g, &pl)) return no("implicit GEMM input tile does not fit in LDS");
  const long long blocks = static_cast<long long>(g.N) * pl.tiles_h * pl.tiles_w * g.G * pl.kt_per_group;
  if (blocks > 0x7fffffffLL || static_cast<long long>(g.G) * pl.kt_per_group > 65535) return no("grid too large");
  return true;
}

hipError_t launch_i8_igemm(const Geom& g0, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                           hipStream_t stream) {
  const Geom g = canonical(g0);
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  IgemmPlan pl;
  if (!make_plan(g, &pl)) return hipErrorInvalidConfiguration;

  IgemmArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.R = g.R; a.S = g.S; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.sh = g.sh; a.sw = g.sw; a.dh = g.dh; a.dw = g.dw;
  a.Cg = g.Cg; a.Kg = g.Kg; a.Cg16 = g.Cg / 16;
  a.NQ = g.R * g.S * a.Cg16;
  a.KB = (a.NQ + 3) / 4;
  a.Kdim = g.R * g.S * g.Cg;
  a.KBC = pl.KBC; a.nchunks = pl.nchunks;
  a.RB = pl.RB; a.CB = pl.CB; a.tiles_h = pl.tiles_h; a.tiles_w = pl.tiles_w;
  a.kt_per_group = pl.kt_per_group;
  const HaloDims hd = halo_dims(g, pl.RB, pl.CB);
  a.HCs = hd.HCs; a.PS = hd.PS; a.nslot = hd.nslot;
  a.fd_ps = make_fastdiv(hd.PS);
  a.fd_hcs = make_fastdiv(hd.HCs);
  a.fd_sw = make_fastdiv(g.sw);
  a.fd_cb = make_fastdiv(pl.CB);
  a.fd_cg16 = make_fastdiv(a.Cg16);
  a.fd_s = make_fastdiv(g.S);
  a.fd_tiles_img = make_fastdiv(pl.tiles_h * pl.tiles_w);
  a.fd_tiles_w = make_fastdiv(pl.tiles_w);
  a.fd_ktpg = make_fastdiv(pl.kt_per_group);
  a.fd_gx = make_fastdiv(g.N * pl.tiles_h * pl.tiles_w);
  a.w_off = pl.w_off; a.h_off = pl.h_off; a.w_buf_bytes = pl.w_buf_bytes;
  a.act_scale = rq.act_scale;
  a.relu = rq.relu;

  switch (epi) {
    case kEpiI8: launch_epi<kEpiI8>(a, pl, g.N, g.G, stream); break;
    case kEpiAcc32: launch_epi<kEpiAcc32>(a, pl, g.N, g.G, stream); break;
    default: launch_epi<kEpiF32>(a, pl, g.N, g.G, stream); break;
  }
  return hipGetLastError();
}

}  // namespace miq
