// int8 convolution on the vector ALU (v_dot4_i32_i8): the bandwidth-bound fallback without
// matrix instructions, for thin-channel layers and layers with few output channels.
//
//   y[n,ho,wo,g*Kg+k] = requant( sum over in-bounds taps (r, s), ci < Cg of
//                                x[n, ho*sh-ph+r*dh, wo*sw-pw+s*dw, g*Cg+ci] * w[g*Kg+k, r, s, ci] )
//
// with int32 wrap-around sums, the arithmetic of every other int8 kernel (i8_direct_kernel).
//
// i8_dot4_kernel.  A thread computes P output pixels x KT consecutive output channels of one
// group; a workgroup of 256 threads takes 256 * P consecutive pixels (pixel i of a thread is
// 256 * i + thread, so every load and store of the 256 threads is one contiguous run) and one
// channel tile.  The channel tile is the fastest index of the launch, so the workgroups that
// read the same input pixels run side by side and share them in L2.
//   - The tile's filter is repacked once into LDS as [tap][c4][KT] dwords (c4: 4 input
//     channels; channels past Cg or Kg are zero), so one 16-byte LDS read gives the weights of
//     4 output channels for one (tap, c4), the same address for every lane (a broadcast).  Each
//     weight read feeds P dot products.
//   - Input: 4 channels of one tap per dword, 16 / P dwords per pixel loaded before their dot
//     products (one memory latency per chunk, 16 dwords in flight per thread).  16-byte loads where Cg % 16 == 0 and
//     the rows are 16-byte aligned, dword loads where Cg % 4 == 0, otherwise the bytes one by
//     one, packed (C = 3).  Taps outside the image contribute nothing (their dwords are zero).
//   - 64 * KT * P / 64 accumulators per thread; the epilogue requantizes each pixel's KT
//     channels and stores them as one run (16-byte stores where they align).

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kDot4Threads = 256;
constexpr int kDot4MaxLds = 64 * 1024;
constexpr int kChunkDwords = 16;  // input dwords a thread loads together (over its P pixels)


struct Dot4Args {
  const int8_t* x;
  const int8_t* w;
  void* y;
  Requant rq;
  Geom g;
  int taps;      // R * S
  int C4;        // ceil(Cg / 4)
  int nkt;       // channel tiles over all groups: G * ceil(Kg / KT)
  int kt_per_g;  // ceil(Kg / KT)
  long long npix;  // N * Ho * Wo
  int aligned;   // Cg % 4 == 0 and C % 4 == 0 and x 4-byte aligned: one dword per (tap, c4)
  int vec16;     // also Cg % 16 == 0, C % 16 == 0 and x 16-byte aligned: 16-byte loads
  FastDiv fd_nkt, fd_ktg, fd_wo, fd_ho;
};

template <int KT, int P, int EPI>
__global__ void __launch_bounds__(kDot4Threads) i8_dot4_kernel(Dot4Args a) {
  extern __shared__ v4i wl[];  // [tap][c4][KT / 4] of 4 dwords
  constexpr int kChunk = kChunkDwords / P;  // dwords (4 channels each) of one tap per pixel and chunk
  const Geom& g = a.g;
  const int lin = blockIdx.x;
  const int pb = fdiv(lin, a.fd_nkt);
  const int kt = lin - pb * a.nkt;
  const int grp = fdiv(kt, a.fd_ktg);
  const int k0 = (kt - grp * a.kt_per_g) * KT;  // first channel of the tile, in group grp
  const int t = threadIdx.x;

  // ---- the tile's filter -> LDS, [tap][c4][j] dwords, zero past Cg or Kg ----
  {
    int* wd = reinterpret_cast<int*>(wl);
    const int total = a.taps * a.C4 * KT;
    const size_t rsc = static_cast<size_t>(a.taps) * g.Cg;
    for (int i = t; i < total; i += kDot4Threads) {
      const int j = i % KT;
      const int tc = i / KT;
      const int c4 = tc % a.C4;
      const int tap = tc / a.C4;
      const int k = k0 + j;
      unsigned v = 0;
      if (k < g.Kg) {
        const int8_t* wp = a.w + static_cast<size_t>(grp * g.Kg + k) * rsc + static_cast<size_t>(tap) * g.Cg;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int ci = 4 * c4 + b;
          if (ci < g.Cg) v |= static_cast<unsigned>(static_cast<unsigned char>(wp[ci])) << (8 * b);
        }
      }
      wd[i] = static_cast<int>(v);
    }
  }
  __syncthreads();

  // ---- this thread's pixels ----
  int hb[P], wb[P];
  const int8_t* xn[P];
  bool live[P];
  long long pix[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    pix[i] = (static_cast<long long>(pb) * P + i) * kDot4Threads + t;
    live[i] = pix[i] < a.npix;
    const int p = static_cast<int>(live[i] ? pix[i] : 0);  // npix < 2^31 (launch check)
    const int q = fdiv(p, a.fd_wo);
    const int wo = p - q * g.Wo;
    const int n = fdiv(q, a.fd_ho);
    const int ho = q - n * g.Ho;
    hb[i] = ho * g.sh - g.ph;
    wb[i] = wo * g.sw - g.pw;
    xn[i] = a.x + static_cast<size_t>(n) * g.H * g.W * g.C + static_cast<size_t>(grp) * g.Cg;
  }

  int acc[P][KT];
#pragma unroll
  for (int i = 0; i < P; ++i)
#pragma unroll
    for (int j = 0; j < KT; ++j) acc[i][j] = 0;

  for (int r = 0; r < g.R; ++r) {
    for (int s = 0; s < g.S; ++s) {
      const int tap = r * g.S + s;
      const int8_t* xp[P];
      bool ok[P];
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int hi = hb[i] + r * g.dh;
        const int wi = wb[i] + s * g.dw;
        ok[i] = live[i] && hi >= 0 && hi < g.H && wi >= 0 && wi < g.W;
        xp[i] = xn[i] + (ok[i] ? (static_cast<size_t>(hi) * g.W + wi) * g.C : 0);
      }
      // chunks of up to kChunk dwords per pixel: every load of a chunk is issued before its
      // dot products, so a chunk costs one memory latency
      for (int cb = 0; cb < a.C4; cb += kChunk) {
        int xv[P][kChunk];
#pragma unroll
        for (int i = 0; i < P; ++i) {
          if (kChunk % 4 == 0 && a.vec16) {  // C4 % 4 == 0: whole 16-byte groups
#pragma unroll
            for (int u = 0; u < kChunk; u += 4) {
              v4i v = v4i{0, 0, 0, 0};
              if (ok[i] && cb + u < a.C4) v = *reinterpret_cast<const v4i*>(xp[i] + 4 * (cb + u));
              xv[i][u] = v[0];
              xv[i][u + 1] = v[1];
              xv[i][u + 2] = v[2];
              xv[i][u + 3] = v[3];
            }
          } else if (a.aligned) {
#pragma unroll
            for (int u = 0; u < kChunk; ++u)
              xv[i][u] = ok[i] && cb + u < a.C4 ? *reinterpret_cast<const int*>(xp[i] + 4 * (cb + u)) : 0;
          } else {
#pragma unroll
            for (int u = 0; u < kChunk; ++u) {
              unsigned v = 0;
              if (ok[i] && cb + u < a.C4) {
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                  const int ci = 4 * (cb + u) + b;
                  if (ci < g.Cg) v |= static_cast<unsigned>(static_cast<unsigned char>(xp[i][ci])) << (8 * b);
                }
              }
              xv[i][u] = static_cast<int>(v);
            }
          }
        }
        const int nu = min(kChunk, a.C4 - cb);
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
          if (u >= nu) break;  // uniform
          const v4i* wrow = wl + (tap * a.C4 + cb + u) * (KT / 4);
#pragma unroll
          for (int jq = 0; jq < KT / 4; ++jq) {
            const v4i wq = wrow[jq];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int i = 0; i < P; ++i)
                acc[i][4 * jq + q] = __builtin_amdgcn_sdot4(xv[i][u], wq[q], acc[i][4 * jq + q], false);
          }
        }
      }
    }
  }

  // ---- epilogue: pixel i's channels k0 .. k0 + KT - 1 of group grp ----
  const int nk = min(KT, g.Kg - k0);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    if (!live[i]) continue;
    const size_t base = static_cast<size_t>(pix[i]) * g.K + static_cast<size_t>(grp) * g.Kg + k0;
    if constexpr (EPI == kEpiAcc32) {
      int32_t* yp = static_cast<int32_t*>(a.y) + base;
#pragma unroll
      for (int j = 0; j < KT; ++j)
        if (j < nk) yp[j] = acc[i][j];
    } else if constexpr (EPI == kEpiI8) {
      int q[KT];
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const int kk = grp * g.Kg + k0 + min(j, nk - 1);
        const int32_t b = a.rq.bias ? a.rq.bias[kk] : 0;
        const float m = requant_multiplier(a.rq.act_scale, a.rq.wscale[kk]);
        q[j] = requant_i8(acc[i][j], b, m, a.rq.relu ? 0.0f : -128.0f);
      }
      int8_t* yp = static_cast<int8_t*>(a.y) + base;
      if (nk == KT && KT % 4 == 0 && (reinterpret_cast<uintptr_t>(yp) & 3u) == 0) {
#pragma unroll
        for (int j = 0; j < KT; j += 4) {
          const unsigned packed = (static_cast<unsigned>(q[j]) & 0xFFu) | ((static_cast<unsigned>(q[j + 1]) & 0xFFu) << 8) |
                                  ((static_cast<unsigned>(q[j + 2]) & 0xFFu) << 16) |
                                  ((static_cast<unsigned>(q[j + 3]) & 0xFFu) << 24);
          *reinterpret_cast<unsigned*>(yp + j) = packed;
        }
      } else {
#pragma unroll
        for (int j = 0; j < KT; ++j)
          if (j < nk) yp[j] = static_cast<int8_t>(q[j]);
      }
    } else {
      float* yp = static_cast<float*>(a.y) + base;
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        if (j >= nk) continue;
        const int kk = grp * g.Kg + k0 + j;
        const int32_t b = a.rq.bias ? a.rq.bias[kk] : 0;
        yp[j] = dequant_f32(acc[i][j], b, requant_multiplier(a.rq.act_scale, a.rq.wscale[kk]), a.rq.relu);
      }
    }
  }
}

// channels per thread for a group of Kg output channels, and pixels per thread: the most
// that still gives the launch at least two workgroups per CU (4 for 4 or 8 channels, 2 for 16,
// 1 for 32)
void dot4_tile(const Geom& g, int* kt, int* p) {
  *kt = g.Kg <= 4 ? 4 : g.Kg <= 8 ? 8 : g.Kg <= 16 ? 16 : 32;
  const long long npix = static_cast<long long>(g.N) * g.Ho * g.Wo;
  const long long nkt = static_cast<long long>(g.G) * ((g.Kg + *kt - 1) / *kt);
  *p = *kt <= 8 ? 4 : *kt == 16 ? 2 : 1;
  while (*p > 1 && ((npix + kDot4Threads * *p - 1) / (kDot4Threads * *p)) * nkt < 512) *p /= 2;
}

template <int KT, int P>
hipError_t dot4_launch(const Dot4Args& a, Epi epi, unsigned blocks, size_t lds, hipStream_t stream) {
  switch (epi) {
    case kEpiI8: hipLaunchKernelGGL((i8_dot4_kernel<KT, P, kEpiI8>), dim3(blocks), dim3(kDot4Threads), lds, stream, a); break;
    case kEpiAcc32: hipLaunchKernelGGL((i8_dot4_kernel<KT, P, kEpiAcc32>), dim3(blocks), dim3(kDot4Threads), lds, stream, a); break;
    default: hipLaunchKernelGGL((i8_dot4_kernel<KT, P, kEpiF32>), dim3(blocks), dim3(kDot4Threads), lds, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace

bool dot4_eligible(const Geom& g, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  int kt, p;
  dot4_tile(g, &kt, &p);
  const long long lds = static_cast<long long>(g.R) * g.S * ((g.Cg + 3) / 4) * kt * 4;
  if (lds > kDot4MaxLds) return no("dot4 kernel: the filter tile (r*s*ceil(c/groups/4)*channels dwords) exceeds 64 KB of LDS");
  const long long npix = static_cast<long long>(g.N) * g.Ho * g.Wo;
  if (npix >= (1LL << 31) - 4LL * kDot4Threads) return no("dot4 kernel: more than 2^31 output pixels");
  const long long blocks = ((npix + kDot4Threads * p - 1) / (kDot4Threads * p)) * g.G * ((g.Kg + kt - 1) / kt);
  if (blocks > (1LL << 31) - 1) return no("dot4 kernel: grid exceeds 2^31 workgroups");
  return true;
}

bool dot4_preferred(const Geom& g) {
  // measured against the implicit GEMM, the kernel AUTO takes otherwise for these shapes:
  // 1x1 with 1-8 output channels per group 1.2-3.1x faster (C/groups 16-512, N 1 and 32),
  // 3x3 16 -> 8 1.2x; equal at 12 channels, slower at 3x3 64 -> 8 and wherever the band
  // kernels apply (16 or more channels per group)
  return g.Kg <= 8 && g.Cg % 4 == 0 && (g.R * g.S == 1 || g.R * g.S * g.Cg <= 144) && dot4_eligible(g, nullptr);
}

hipError_t launch_i8_dot4(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream) {
  int kt, p;
  dot4_tile(g, &kt, &p);
  Dot4Args a;
  a.x = x; a.w = w; a.y = y; a.rq = rq; a.g = g;
  a.taps = g.R * g.S;
  a.C4 = (g.Cg + 3) / 4;
  a.kt_per_g = (g.Kg + kt - 1) / kt;
  a.nkt = g.G * a.kt_per_g;
  a.npix = static_cast<long long>(g.N) * g.Ho * g.Wo;
  a.aligned = g.Cg % 4 == 0 && g.C % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 3u) == 0;
  a.vec16 = g.Cg % 16 == 0 && g.C % 16 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  a.fd_nkt = make_fastdiv(static_cast<uint32_t>(a.nkt));
  a.fd_ktg = make_fastdiv(static_cast<uint32_t>(a.kt_per_g));
  a.fd_wo = make_fastdiv(static_cast<uint32_t>(g.Wo));
  a.fd_ho = make_fastdiv(static_cast<uint32_t>(g.Ho));
  if (a.npix == 0 || a.nkt == 0) return hipSuccess;
  const long long pblocks = (a.npix + static_cast<long long>(kDot4Threads) * p - 1) / (static_cast<long long>(kDot4Threads) * p);
  const unsigned blocks = static_cast<unsigned>(pblocks * a.nkt);
  const size_t lds = static_cast<size_t>(a.taps) * a.C4 * kt * 4;
  switch (kt * 8 + p) {
    case 4 * 8 + 4: return dot4_launch<4, 4>(a, epi, blocks, lds, stream);
    case 4 * 8 + 2: return dot4_launch<4, 2>(a, epi, blocks, lds, stream);
    case 4 * 8 + 1: return dot4_launch<4, 1>(a, epi, blocks, lds, stream);
    case 8 * 8 + 4: return dot4_launch<8, 4>(a, epi, blocks, lds, stream);
    case 8 * 8 + 2: return dot4_launch<8, 2>(a, epi, blocks, lds, stream);
    case 8 * 8 + 1: return dot4_launch<8, 1>(a, epi, blocks, lds, stream);
    case 16 * 8 + 2: return dot4_launch<16, 2>(a, epi, blocks, lds, stream);
    case 16 * 8 + 1: return dot4_launch<16, 1>(a, epi, blocks, lds, stream);
    default: return dot4_launch<32, 1>(a, epi, blocks, lds, stream);
  }
}

}  // namespace miq
