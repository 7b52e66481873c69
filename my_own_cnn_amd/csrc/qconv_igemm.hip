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
// Work decomposition: a workgroup (4 waves) owns one tile of RB output rows x CB output
// columns of one image and 64*NKT*WAVES_K output channels of one group.  The input
// patch the tile needs (its "halo": rows*stride + dilated taps, all Cg channels) is
// staged once into LDS with coalesced 16-byte loads, zero-filled where the convolution
// pads; every tap then reads shifted windows of it.  16-byte chunks are XOR-swizzled
// within a pixel so that the 16 lanes of a group reading 16 neighbouring pixels hit
// distinct LDS banks.

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kThreads = 256;
constexpr int kLdsBudget = 64 * 1024;  // bytes of dynamic LDS per workgroup

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
  int RB, CB;        // output tile extent
  int tiles_h, tiles_w;
  int kt_per_group;  // channel tiles (of 64*NKT*WAVES_K) per group
  int swz_shift, swz_mask;
  float act_scale;
  int relu;
};

__device__ __forceinline__ int swz(int hp, int shift, int mask) {
  return ((hp >> shift) ^ (hp >> (shift + 3))) & mask;
}

template <int NKT, int NSEG, int WAVES_K, int EPI>
__global__ void __launch_bounds__(kThreads)
i8_igemm_kernel(IgemmArgs a) {
  constexpr int WAVES_P = 4 / WAVES_K;
  constexpr int KTILE = 64 * NKT;  // output channels per wave
  extern __shared__ v4i halo[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wk = wave % WAVES_K;
  const int wp = wave / WAVES_K;

  const int tiles_img = a.tiles_h * a.tiles_w;
  const int n = blockIdx.x / tiles_img;
  const int trem = blockIdx.x - n * tiles_img;
  const int th = trem / a.tiles_w;
  const int tw = trem - th * a.tiles_w;
  const int gi = blockIdx.y / a.kt_per_group;
  const int kt = blockIdx.y - gi * a.kt_per_group;

  const int ho0 = th * a.RB;
  const int wo0 = tw * a.CB;
  const int rows = min(a.RB, a.Ho - ho0);
  const int cols = min(a.CB, a.Wo - wo0);
  const int HR = (rows - 1) * a.sh + (a.R - 1) * a.dh + 1;
  const int HC = (cols - 1) * a.sw + (a.S - 1) * a.dw + 1;
  const int hi0 = ho0 * a.sh - a.ph;
  const int wi0 = wo0 * a.sw - a.pw;

  // ---- stage the input halo of this tile (this group's channels) into LDS ----
  const int8_t* xg = a.x + static_cast<size_t>(n) * a.H * a.W * a.C + static_cast<size_t>(gi) * a.Cg;
  const int nchunk = HR * HC * a.Cg16;
  for (int i = tid; i < nchunk; i += kThreads) {
    const int hp = i / a.Cg16;
    const int c16 = i - hp * a.Cg16;
    const int hr = hp / HC;
    const int hc = hp - hr * HC;
    const int hi = hi0 + hr;
    const int wi = wi0 + hc;
    v4i v = {0, 0, 0, 0};
    if (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) && static_cast<unsigned>(wi) < static_cast<unsigned>(a.W)) {
      v = *reinterpret_cast<const v4i*>(xg + (static_cast<size_t>(hi) * a.W + wi) * a.C + c16 * 16);
    }
    halo[hp * a.Cg16 + (c16 ^ swz(hp, a.swz_shift, a.swz_mask))] = v;
  }
  __syncthreads();

  const int kwave0 = kt * (KTILE * WAVES_K) + wk * KTILE;  // first channel of this wave within the group
  if (kwave0 >= a.Kg) return;                               // no barrier follows

  const int npix = rows * cols;
  const int nseg = (npix + 15) >> 4;
  const int row_l = lane & 15;  // MFMA row (A) / column (B) of this lane
  const int grp_l = lane >> 4;  // chunk slot of this lane inside a K-block
  const int8_t* wg = a.w + static_cast<size_t>(gi) * a.Kg * a.Kdim;

  // Filter rows this lane feeds to the A operand of MFMA (t, j).
  int kc[NKT][4];
#pragma unroll
  for (int t = 0; t < NKT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) kc[t][j] = kwave0 + t * 64 + 16 * (row_l >> 2) + 4 * j + (row_l & 3);

  for (int sg0 = wp * NSEG; sg0 < nseg; sg0 += WAVES_P * NSEG) {
    int pb[NSEG];
    bool pv[NSEG];
#pragma unroll
    for (int i = 0; i < NSEG; ++i) {
      const int p = (sg0 + i) * 16 + row_l;
      pv[i] = p < npix;
      const int lho = p / cols;
      const int lwo = p - lho * cols;
      pb[i] = pv[i] ? (lho * a.sh) * HC + lwo * a.sw : 0;
    }

    v4i acc[NKT][4][NSEG];
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < NSEG; ++i) acc[t][j][i] = v4i{0, 0, 0, 0};

    for (int b = 0; b < a.KB; ++b) {
      const int q = 4 * b + grp_l;
      const bool qv = q < a.NQ;
      const int tap = q / a.Cg16;
      const int c16 = q - tap * a.Cg16;
      const int rr = tap / a.S;
      const int ss = tap - rr * a.S;
      const int toff = rr * a.dh * HC + ss * a.dw;

      v4i A[NKT][4];
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v4i v = {0, 0, 0, 0};
          if (qv && kc[t][j] < a.Kg) v = *reinterpret_cast<const v4i*>(wg + static_cast<size_t>(kc[t][j]) * a.Kdim + q * 16);
          A[t][j] = v;
        }
      v4i B[NSEG];
#pragma unroll
      for (int i = 0; i < NSEG; ++i) {
        const int hp = pb[i] + toff;
        v4i v = {0, 0, 0, 0};
        if (qv && pv[i]) v = halo[hp * a.Cg16 + (c16 ^ swz(hp, a.swz_shift, a.swz_mask))];
        B[i] = v;
      }
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < NSEG; ++i)
            acc[t][j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[t][j], B[i], acc[t][j][i], 0, 0, 0);
    }

    // ---- epilogue: lane holds channels kc0 .. kc0+15 of pixel p for each (t, i) ----
    const Requant rq{a.bias, a.wscale, a.act_scale, a.relu};
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
      const int kc0 = kwave0 + t * 64 + 16 * grp_l;
      if (kc0 >= a.Kg) continue;
      const int kabs = gi * a.Kg + kc0;
      const bool full = (kc0 + 16 <= a.Kg) && ((a.Kg & 15) == 0);
      int32_t bv[16];
      float mv[16];
      load_requant16<EPI>(rq, kc0, a.Kg, kabs, bv, mv);
#pragma unroll
      for (int i = 0; i < NSEG; ++i) {
        if (!pv[i]) continue;
        const int p = (sg0 + i) * 16 + row_l;
        const int lho = p / cols;
        const int lwo = p - lho * cols;
        const size_t opix = (static_cast<size_t>(n) * a.Ho + (ho0 + lho)) * a.Wo + (wo0 + lwo);
        const v4i frag[4] = {acc[t][0][i], acc[t][1][i], acc[t][2][i], acc[t][3][i]};
        store16<EPI>(a.y, opix * a.K + kabs, frag, kc0, a.Kg, full, bv, mv, a.relu);
      }
    }
  }
}

// Host-side tiling decision for one problem.
struct IgemmPlan {
  int nkt, waves_k, nseg;
  int RB, CB, tiles_h, tiles_w, kt_per_group;
  size_t lds_bytes;
};

size_t halo_bytes(const Geom& g, int RB, int CB) {
  const size_t HR = static_cast<size_t>(RB - 1) * g.sh + static_cast<size_t>(g.R - 1) * g.dh + 1;
  const size_t HC = static_cast<size_t>(CB - 1) * g.sw + static_cast<size_t>(g.S - 1) * g.dw + 1;
  return HR * HC * static_cast<size_t>(g.Cg);
}

bool make_plan(const Geom& g, IgemmPlan* pl) {
  // Channel tiling: one wave covers 64*nkt channels; waves_k waves split the channels.
  if (g.Kg <= 64) {
    pl->nkt = 1; pl->waves_k = 1;
  } else if (g.Kg <= 128) {
    pl->nkt = 1; pl->waves_k = 2;
  } else if (g.Kg <= 256) {
    pl->nkt = 1; pl->waves_k = 4;
  } else {
    pl->nkt = 2; pl->waves_k = 4;
  }
  pl->nseg = 4;
  const int waves_p = 4 / pl->waves_k;
  const int tp = waves_p * pl->nseg * 16;  // pixels per tile
  pl->kt_per_group = (g.Kg + 64 * pl->nkt * pl->waves_k - 1) / (64 * pl->nkt * pl->waves_k);

  // Spatial tiling: whole output rows when they are short, otherwise row segments.
  int CB = std::min(g.Wo, tp);
  int RB = std::max(1, tp / CB);
  RB = std::min(RB, g.Ho);
  while (RB > 1 && halo_bytes(g, RB, CB) > static_cast<size_t>(kLdsBudget)) --RB;
  while (CB > 16 && halo_bytes(g, RB, CB) > static_cast<size_t>(kLdsBudget)) CB -= 16;
  if (halo_bytes(g, RB, CB) > static_cast<size_t>(kLdsBudget)) return false;
  pl->RB = RB;
  pl->CB = CB;
  pl->tiles_h = (g.Ho + RB - 1) / RB;
  pl->tiles_w = (g.Wo + CB - 1) / CB;
  pl->lds_bytes = halo_bytes(g, RB, CB);
  return true;
}

template <int NKT, int WAVES_K, int EPI>
void launch_cfg(const IgemmArgs& a, const IgemmPlan& pl, int N, int G, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(N * pl.tiles_h * pl.tiles_w), static_cast<unsigned>(G * pl.kt_per_group));
  hipLaunchKernelGGL((i8_igemm_kernel<NKT, 4, WAVES_K, EPI>), grid, dim3(kThreads), pl.lds_bytes, stream, a);
}

template <int EPI>
void launch_epi(const IgemmArgs& a, const IgemmPlan& pl, int N, int G, hipStream_t stream) {
  if (pl.nkt == 2) {
    launch_cfg<2, 4, EPI>(a, pl, N, G, stream);
  } else if (pl.waves_k == 4) {
    launch_cfg<1, 4, EPI>(a, pl, N, G, stream);
  } else if (pl.waves_k == 2) {
    launch_cfg<1, 2, EPI>(a, pl, N, G, stream);
  } else {
    launch_cfg<1, 1, EPI>(a, pl, N, G, stream);
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
  const long long grid_x = static_cast<long long>(g.N) * pl.tiles_h * pl.tiles_w;
  if (grid_x > 0x7fffffffLL || static_cast<long long>(g.G) * pl.kt_per_group > 65535) return no("grid too large");
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
  a.RB = pl.RB; a.CB = pl.CB; a.tiles_h = pl.tiles_h; a.tiles_w = pl.tiles_w;
  a.kt_per_group = pl.kt_per_group;
  if (a.Cg16 % 8 == 0) {
    a.swz_shift = 0; a.swz_mask = 7;
  } else if (a.Cg16 % 4 == 0) {
    a.swz_shift = 1; a.swz_mask = 3;
  } else if (a.Cg16 % 2 == 0) {
    a.swz_shift = 2; a.swz_mask = 1;
  } else {
    a.swz_shift = 0; a.swz_mask = 0;
  }
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
