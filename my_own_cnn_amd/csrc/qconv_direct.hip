// Direct (VALU) convolution kernels: the compat int32 path on float codes with
// per-sample zero points, and the int8 fallback for shapes the MFMA kernels do not take.
//
// One thread computes one output element; consecutive threads take consecutive output
// channels of one pixel, so the stores are coalesced and the input taps of a pixel are
// shared through the L1 cache by the threads of its channels.

#include "qconv_internal.h"

namespace miq {
namespace {

constexpr int kThreads = 256;

// Per-sample zero point, read from the raw parameter struct the caller copied to the
// device: uint8 at offset 0 of a 12-byte struct (LinQuantU8), int8 at offset 0 of an
// 8-byte struct (LinQuantS5).
template <QpKind Q>
__device__ __forceinline__ int zero_point_at(const unsigned char* qp, int i) {
  if constexpr (Q == kQpU8) {
    return static_cast<int>(qp[static_cast<size_t>(i) * 12]);
  } else {
    return static_cast<int>(static_cast<signed char>(qp[static_cast<size_t>(i) * 8]));
  }
}

// Follows the accumulation of cpu_fprop_nhwc_qi32_impl / cpu_block_fprop_nhwc_qi32_impl
// (/root/reference/src/cpu_ref.cpp:36-112): codes are truncated to int32, centred by the
// sample's (input) and the filter's zero point, and padded taps are skipped.
template <QpKind Q, bool BLOCKED>
__global__ void __launch_bounds__(kThreads)
qi32_direct_kernel(const float* __restrict__ x, const float* __restrict__ w, int32_t* __restrict__ y,
                   const unsigned char* __restrict__ in_qp, const unsigned char* __restrict__ f_qp,
                   Geom g, BlockGeom bg, long long total) {
  const long long e = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= total) return;
  const int k = static_cast<int>(e % g.K);
  const long long pix = e / g.K;
  const int wo = static_cast<int>(pix % g.Wo);
  const long long t = pix / g.Wo;
  const int ho = static_cast<int>(t % g.Ho);
  const int n = static_cast<int>(t / g.Ho);
  const int grp = k / g.Kg;

  const int zx = zero_point_at<Q>(in_qp, n);
  const int zw = zero_point_at<Q>(f_qp, 0);
  const size_t taps = static_cast<size_t>(g.R) * g.S * g.Cg;
  const float* wk;
  if constexpr (BLOCKED) {
    const int by = ho / bg.bho;
    const int bx = wo / bg.bwo;
    wk = w + ((static_cast<size_t>(k) * bg.By + by) * bg.Bx + bx) * taps;
  } else {
    wk = w + static_cast<size_t>(k) * taps;
  }

  uint32_t acc = 0;  // two's-complement wrap-around, no signed-overflow UB
  for (int r = 0; r < g.R; ++r) {
    const int hi = ho * g.sh - g.ph + r * g.dh;
    if (hi < 0 || hi >= g.H) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wi = wo * g.sw - g.pw + s * g.dw;
      if (wi < 0 || wi >= g.W) continue;
      const float* xp = x + ((static_cast<size_t>(n) * g.H + hi) * g.W + wi) * g.C + static_cast<size_t>(grp) * g.Cg;
      const float* wp = wk + (static_cast<size_t>(r) * g.S + s) * g.Cg;
      for (int ci = 0; ci < g.Cg; ++ci) {
        const int32_t xv = static_cast<int32_t>(xp[ci]) - zx;
        const int32_t wv = static_cast<int32_t>(wp[ci]) - zw;
        acc += static_cast<uint32_t>(xv) * static_cast<uint32_t>(wv);
      }
    }
  }
  y[e] = static_cast<int32_t>(acc);
}

// int8 codes, zero points 0, fused output stage.
template <int EPI>
__global__ void __launch_bounds__(kThreads)
i8_direct_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ w, void* __restrict__ y,
                 Geom g, Requant rq, long long total) {
  const long long e = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= total) return;
  const int k = static_cast<int>(e % g.K);
  const long long pix = e / g.K;
  const int wo = static_cast<int>(pix % g.Wo);
  const long long t = pix / g.Wo;
  const int ho = static_cast<int>(t % g.Ho);
  const int n = static_cast<int>(t / g.Ho);
  const int grp = k / g.Kg;
  const int8_t* wk = w + static_cast<size_t>(k) * g.R * g.S * g.Cg;

  uint32_t acc = 0;
  for (int r = 0; r < g.R; ++r) {
    const int hi = ho * g.sh - g.ph + r * g.dh;
    if (hi < 0 || hi >= g.H) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wi = wo * g.sw - g.pw + s * g.dw;
      if (wi < 0 || wi >= g.W) continue;
      const int8_t* xp = x + ((static_cast<size_t>(n) * g.H + hi) * g.W + wi) * g.C + static_cast<size_t>(grp) * g.Cg;
      const int8_t* wp = wk + (static_cast<size_t>(r) * g.S + s) * g.Cg;
      for (int ci = 0; ci < g.Cg; ++ci) {
        acc += static_cast<uint32_t>(static_cast<int32_t>(xp[ci]) * static_cast<int32_t>(wp[ci]));
      }
    }
  }

  const int32_t a = static_cast<int32_t>(acc);
  if constexpr (EPI == kEpiAcc32) {
    static_cast<int32_t*>(y)[e] = a;
  } else {
    const int32_t b = rq.bias ? rq.bias[k] : 0;
    const float m = requant_multiplier(rq.act_scale, rq.wscale[k]);
    if constexpr (EPI == kEpiI8) {
      static_cast<int8_t*>(y)[e] = static_cast<int8_t>(requant_i8(a, b, m, rq.relu ? 0.0f : -128.0f));
    } else {
      static_cast<float*>(y)[e] = dequant_f32(a, b, m, rq.relu);
    }
  }
}

unsigned grid_for(long long total) {
  return static_cast<unsigned>((total + kThreads - 1) / kThreads);
}

}  // namespace

hipError_t launch_qi32_direct(const Geom& g, const BlockGeom& bg, QpKind qp, const float* x, const float* w,
                              int32_t* y, const void* in_qp, const void* f_qp, hipStream_t stream) {
  const long long total = static_cast<long long>(g.N) * g.Ho * g.Wo * g.K;
  if (total == 0) return hipSuccess;
  const bool blocked = (bg.By != 1 || bg.Bx != 1);
  const auto* iq = static_cast<const unsigned char*>(in_qp);
  const auto* fq = static_cast<const unsigned char*>(f_qp);
  const dim3 grid(grid_for(total)), block(kThreads);
  if (qp == kQpU8) {
    if (blocked) {
      hipLaunchKernelGGL((qi32_direct_kernel<kQpU8, true>), grid, block, 0, stream, x, w, y, iq, fq, g, bg, total);
    } else {
      hipLaunchKernelGGL((qi32_direct_kernel<kQpU8, false>), grid, block, 0, stream, x, w, y, iq, fq, g, bg, total);
    }
  } else {
    if (blocked) {
      hipLaunchKernelGGL((qi32_direct_kernel<kQpS5, true>), grid, block, 0, stream, x, w, y, iq, fq, g, bg, total);
    } else {
      hipLaunchKernelGGL((qi32_direct_kernel<kQpS5, false>), grid, block, 0, stream, x, w, y, iq, fq, g, bg, total);
    }
  }
  return hipGetLastError();
}

hipError_t launch_i8_direct(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                            hipStream_t stream) {
  const long long total = static_cast<long long>(g.N) * g.Ho * g.Wo * g.K;
  if (total == 0) return hipSuccess;
  const dim3 grid(grid_for(total)), block(kThreads);
  switch (epi) {
    case kEpiI8:
      hipLaunchKernelGGL((i8_direct_kernel<kEpiI8>), grid, block, 0, stream, x, w, y, g, rq, total);
      break;
    case kEpiAcc32:
      hipLaunchKernelGGL((i8_direct_kernel<kEpiAcc32>), grid, block, 0, stream, x, w, y, g, rq, total);
      break;
    default:
      hipLaunchKernelGGL((i8_direct_kernel<kEpiF32>), grid, block, 0, stream, x, w, y, g, rq, total);
      break;
  }
  return hipGetLastError();
}

}  // namespace miq
