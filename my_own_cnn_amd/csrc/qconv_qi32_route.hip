// int32 convolution on quantized float codes (the reference's launch_fprop_nhwc_qi32<Tin>,
// /root/reference/src/conv_types.h:308-323 -> cuda_kernels.cu:1336-1392) through the int8
// stream kernel, for the shapes it takes (strided rows, filters too large for registers).
// The result is the reference's CPU definition (cpu_ref.cpp:36-72):
//   y[n,ho,wo,g*Kg+k] = sum over in-bounds taps (int32(x) - zx[n]) * (int32(w) - zw)
// with int32 wrap-around and int32() truncating toward zero.
//
// Offset codes, as in the row-band kernel: x' = int32(x) - o, w' = int32(w) - o (o = 128 for
// LinQuantU8, 0 for LinQuantS5), a padded tap staged as zx - o so that it contributes nothing.
// With dx = o - zx, dw = o - zw and Kdim = R*S*(C/groups) terms per window (mod 2^32):
//   y = sum x'w' + dx * T(k) + Kdim * dx * dw + dw * W(p)
// (T(k): filter row k's sum; W(p): the pixel's window sum, summed inside the stream kernel
// from the same fragments its MFMAs read).
//
// Three launches per call:
//   1. qi32_route_prep_kernel: blocks [0, nfb) convert the filter (KRSC int8 w' and T), block 0
//      also writes each image's {dx, dw, Kdim * dx * dw}; blocks [nfb, ..) write the input as a
//      padded int8 image (x', padding zx - o), so the stream kernel runs without padding.
//      Each block writes 1 to its flag when a value lies outside int8.
//   2. the stream kernel (kEpiQi32) on the padded image.
//   3. qi32_route_fallback_kernel: every workgroup ORs the flags; unless one is set it exits at
//      once, else the grid recomputes every output directly from the float codes (exact).
//
// The stem route (stride-2 layers with 1..4 channels) is the same scheme on the space-to-depth
// stem kernel: qi32_stem_prep_kernel writes the image as rows of Wq pixels (Wq >= W + 2 pw,
// Wq * C a multiple of 16 bytes, every byte past the image zx - o) and the filter value by
// value (Kdim need not be a multiple of 4); the s2d kernel in its int32 mode sums W(p) from its
// own fragments under a mask of the filter's taps; the same flag pass follows.

#include "qconv_device.h"

#include <algorithm>
#include <type_traits>

namespace miq {
namespace {

constexpr int kRtThreads = 256;

template <QpKind Q>
__device__ __forceinline__ int rt_zero_point(const unsigned char* qp, int i) {
  if constexpr (Q == kQpU8) {
    return static_cast<int>(qp[static_cast<size_t>(i) * 12]);
  } else {
    return static_cast<int>(static_cast<signed char>(qp[static_cast<size_t>(i) * 8]));
  }
}

// 4 codes -> 4 offset int8 values in one word; `bad` is set when one lies outside int8.
__device__ __forceinline__ unsigned rt_pack4(const v4f& v, bool valid, unsigned off, unsigned pad, int& sum,
                                            bool& bad) {
  unsigned word = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const unsigned u = valid ? static_cast<unsigned>(static_cast<int32_t>(v[e])) - off : pad;
    bad |= (u + 128u) > 255u;
    sum += static_cast<int>(u);
    word |= (u & 0xffu) << (8 * e);
  }
  return word;
}

struct RoutePrepArgs {
  const float* x;
  const float* w;
  const unsigned char* in_qp;
  const unsigned char* f_qp;
  int8_t* xp;      // [N][Hp][Wp][C]
  int8_t* wq;      // [K][Kdim]
  int32_t* T;      // [K]
  int32_t* qrec;   // [N][4]
  int32_t* flags;  // [nfb + nib]
  int N, H, W, C, K, Kdim, ph, pw, Hp, Wp;
  int nfb;         // filter blocks: 8 channels each
  long long nchunks;  // input 16-channel chunks: N * Hp * Wp * C / 16
};

template <QpKind Q>
__global__ void __launch_bounds__(kRtThreads) qi32_route_prep_kernel(RoutePrepArgs a) {
  constexpr unsigned kOff = Q == kQpU8 ? 128u : 0u;
  const int t = threadIdx.x;
  bool bad = false;
  if (static_cast<int>(blockIdx.x) < a.nfb) {
    // ---- filter: channel c = 8 * block + t / 32, its float4s q = t % 32 + 32 i ----
    const int c = 8 * static_cast<int>(blockIdx.x) + (t >> 5);
    const int p = t & 31;
    const int nq = a.Kdim / 4;
    int sum = 0;
    if (c < a.K) {
      // 8 loads in flight per batch (buffer loads: only vmcnt counts them, so the waits are exact)
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(c) * a.Kdim, a.Kdim * 4);
      unsigned* out = reinterpret_cast<unsigned*>(a.wq + static_cast<size_t>(c) * a.Kdim);
      for (int q0 = p; q0 < nq; q0 += 32 * 8) {
        v4f v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rw, static_cast<unsigned>(16 * (q0 + 32 * i)), 0, 0));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int q = q0 + 32 * i;
          if (q < nq) out[q] = rt_pack4(v[i], true, kOff, 0u, sum, bad);
        }
      }
    }
    // the 32 lanes of a channel are one half of a wave
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    sum += __shfl_xor(sum, 8);
    sum += __shfl_xor(sum, 16);
    if (p == 0 && c < a.K) a.T[c] = sum;
    if (blockIdx.x == 0) {
      const unsigned dw = kOff - static_cast<unsigned>(rt_zero_point<Q>(a.f_qp, 0));
      for (int n = t; n < a.N; n += kRtThreads) {
        const unsigned dx = kOff - static_cast<unsigned>(rt_zero_point<Q>(a.in_qp, n));
        const v4i rec = {static_cast<int>(dx), static_cast<int>(dw),
                         static_cast<int>(static_cast<unsigned>(a.Kdim) * dx * dw), 0};
        *reinterpret_cast<v4i*>(a.qrec + 4 * n) = rec;
      }
    }
  } else {
    // ---- input: 16 channels of one padded pixel per thread ----
    const long long e = static_cast<long long>(blockIdx.x - a.nfb) * kRtThreads + t;
    if (e < a.nchunks) {
      const int cpp = a.C / 16;
      const long long pix = e / cpp;
      const int ch = static_cast<int>(e - pix * cpp) * 16;
      const int wp = static_cast<int>(pix % a.Wp);
      const long long r = pix / a.Wp;
      const int hp = static_cast<int>(r % a.Hp);
      const int n = static_cast<int>(r / a.Hp);
      const int hi = hp - a.ph;
      const int wi = wp - a.pw;
      const bool ok = hi >= 0 && hi < a.H && wi >= 0 && wi < a.W;
      const unsigned pad = static_cast<unsigned>(rt_zero_point<Q>(a.in_qp, n)) - kOff;
      const float* src = a.x + ((static_cast<size_t>(n) * a.H + (ok ? hi : 0)) * a.W + (ok ? wi : 0)) * a.C + ch;
      v4f v[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) v[d] = *reinterpret_cast<const v4f*>(src + 4 * d);
      v4i o;
      int unused = 0;
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] = static_cast<int>(rt_pack4(v[d], ok, kOff, pad, unused, bad));
      *reinterpret_cast<v4i*>(a.xp + static_cast<size_t>(pix) * a.C + ch) = o;
      store_gap(o);
    }
  }
  const int any = __syncthreads_or(bad ? 1 : 0);
  if (t == 0) a.flags[blockIdx.x] = any ? 1 : 0;
}

struct RouteFallbackArgs {
  const float* x;
  const float* w;
  int32_t* y;
  const unsigned char* in_qp;
  const unsigned char* f_qp;
  const int32_t* flags;
  int nflags;
  Geom g;
  long long total;
};

// Exits at once unless a prepass block flagged a value outside int8; then the grid recomputes
// every output in the reference's loop order (codes truncated, centred, padded taps skipped).
template <QpKind Q>
__global__ void __launch_bounds__(kRtThreads) qi32_route_fallback_kernel(RouteFallbackArgs a) {
  // the flags in 16-byte loads, eight in flight per thread (a loop of dependent 4-byte loads
  // paid one L2 round trip per flag group); the scalar tail and unaligned workspaces word by word
  int any = 0;
  const bool vec = (reinterpret_cast<uintptr_t>(a.flags) & 15u) == 0;
  const int nv = vec ? a.nflags >> 2 : 0;
  const v4i* f4 = reinterpret_cast<const v4i*>(a.flags);
  for (int i0 = threadIdx.x; i0 < nv; i0 += 8 * kRtThreads) {
    v4i f[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kRtThreads;
      f[u] = i < nv ? f4[i] : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) any |= f[u][0] | f[u][1] | f[u][2] | f[u][3];
  }
  for (int i = 4 * nv + static_cast<int>(threadIdx.x); i < a.nflags; i += kRtThreads) any |= a.flags[i];
  if (!__syncthreads_or(any)) return;
  const Geom& g = a.g;
  const int zw = rt_zero_point<Q>(a.f_qp, 0);
  const long long stride = static_cast<long long>(gridDim.x) * kRtThreads;
  for (long long e = static_cast<long long>(blockIdx.x) * kRtThreads + threadIdx.x; e < a.total; e += stride) {
    const int k = static_cast<int>(e % g.K);
    const long long pix = e / g.K;
    const int wo = static_cast<int>(pix % g.Wo);
    const long long tt = pix / g.Wo;
    const int ho = static_cast<int>(tt % g.Ho);
    const int n = static_cast<int>(tt / g.Ho);
    const int grp = k / g.Kg;
    const int zx = rt_zero_point<Q>(a.in_qp, n);
    const float* wk = a.w + static_cast<size_t>(k) * g.R * g.S * g.Cg;
    uint32_t acc = 0;
    for (int r = 0; r < g.R; ++r) {
      const int hi = ho * g.sh - g.ph + r * g.dh;
      if (hi < 0 || hi >= g.H) continue;
      for (int s = 0; s < g.S; ++s) {
        const int wi = wo * g.sw - g.pw + s * g.dw;
        if (wi < 0 || wi >= g.W) continue;
        const float* xp = a.x + ((static_cast<size_t>(n) * g.H + hi) * g.W + wi) * g.C + static_cast<size_t>(grp) * g.Cg;
        const float* wp = wk + (static_cast<size_t>(r) * g.S + s) * g.Cg;
        for (int ci = 0; ci < g.Cg; ++ci) {
          const int32_t xv = static_cast<int32_t>(xp[ci]) - zx;
          const int32_t wv = static_cast<int32_t>(wp[ci]) - zw;
          acc += static_cast<uint32_t>(xv) * static_cast<uint32_t>(wv);
        }
      }
    }
    a.y[e] = static_cast<int32_t>(acc);
  }
}

// ---- the stem route (thin-channel stride-2 layers, the space-to-depth stem kernel): the
// image into rows of Wq pixels (Wq >= W + 2 pw, Wq * C a multiple of 16 bytes), padded taps at
// zx - o; the filter value by value ----
struct StemPrepArgs {
  const float* x;
  const float* w;
  const unsigned char* in_qp;
  const unsigned char* f_qp;
  int8_t* xp;      // [N][Hp][Wq][C]
  int8_t* wq;      // [K][Kdim]
  int32_t* T;      // [K]
  int32_t* qrec;   // [N][4]
  int32_t* flags;  // [nfb + nib]
  int N, H, W, C, K, Kdim, ph, pw, Hp, cpr;  // cpr: 16-byte chunks per padded row (Wq * C / 16)
  int nfb;                                   // filter blocks: 4 channels each
  long long nchunks;                         // N * Hp * cpr 16-byte chunks of the padded input
};


template <QpKind Q>
__global__ void __launch_bounds__(kRtThreads) qi32_stem_prep_kernel(StemPrepArgs a) {
  constexpr unsigned kOff = Q == kQpU8 ? 128u : 0u;
  const int t = threadIdx.x;
  bool bad = false;
  if (static_cast<int>(blockIdx.x) < a.nfb) {
    // ---- filter: channel c = 4 * block + t / 64, its codes t % 64, + 64, ... ----
    const int c = 4 * static_cast<int>(blockIdx.x) + (t >> 6);
    const int l = t & 63;
    int sum = 0;
    if (c < a.K) {
      const float* src = a.w + static_cast<size_t>(c) * a.Kdim;
      int8_t* dst = a.wq + static_cast<size_t>(c) * a.Kdim;
      // four codes per lane in flight before the first conversion (the byte stores may alias
      // the loads as far as the compiler knows, so a plain loop ran one load round trip each)
      for (int i0 = l; i0 < a.Kdim; i0 += 4 * 64) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = i0 + 64 * u < a.Kdim ? src[i0 + 64 * u] : 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = i0 + 64 * u;
          if (i < a.Kdim) {
            const unsigned q = static_cast<unsigned>(static_cast<int32_t>(v[u])) - kOff;
            bad |= (q + 128u) > 255u;
            sum += static_cast<int>(q);
            dst[i] = static_cast<int8_t>(q & 0xffu);
          }
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
    if (l == 0 && c < a.K) a.T[c] = sum;
    if (blockIdx.x == 0) {
      const unsigned dw = kOff - static_cast<unsigned>(rt_zero_point<Q>(a.f_qp, 0));
      for (int n = t; n < a.N; n += kRtThreads) {
        const unsigned dx = kOff - static_cast<unsigned>(rt_zero_point<Q>(a.in_qp, n));
        const v4i rec = {static_cast<int>(dx), static_cast<int>(dw),
                         static_cast<int>(static_cast<unsigned>(a.Kdim) * dx * dw), 0};
        *reinterpret_cast<v4i*>(a.qrec + 4 * n) = rec;
      }
    }
  } else {
    // ---- input: a thread per 16-byte chunk c of padded row `row` (= n * Hp + hp): byte b is
    // code (16c + b - pw C) of image row hp - ph where that lies in the image, else zx - o.
    // With rows of whole float4s the 16 codes come from the five aligned float4s around them
    // (neighbouring threads share the lines), picked at the offset (-pw C) mod 4 every chunk
    // shares; other rows read code by code ----
    const long long idx = static_cast<long long>(static_cast<int>(blockIdx.x) - a.nfb) * kRtThreads + t;
    if (idx < a.nchunks) {
      const int row = static_cast<int>(idx / a.cpr);
      const int c = static_cast<int>(idx - static_cast<long long>(row) * a.cpr);
      const int hp = row % a.Hp;
      const int n = row / a.Hp;
      const int hi = hp - a.ph;
      const int rowb = a.W * a.C;
      const int lead = a.pw * a.C;
      const unsigned pad = static_cast<unsigned>(rt_zero_point<Q>(a.in_qp, n)) - kOff;
      const bool row_ok = hi >= 0 && hi < a.H;
      const int b0 = 16 * c - lead;  // code index of byte 0
      const float* src = a.x + (static_cast<size_t>(n) * a.H + (row_ok ? hi : 0)) * rowb;
      unsigned word[4];
      if (row_ok && (rowb & 3) == 0) {
        const int f0 = b0 >= 0 ? b0 >> 2 : -((3 - b0) >> 2);  // floor(b0 / 4)
        const int nq = rowb >> 2;
        v4f v[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) {
          const int q = f0 + k;
          v[k] = (q >= 0 && q < nq) ? *reinterpret_cast<const v4f*>(src + 4 * q) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
        const int sh = b0 - 4 * f0;  // 0 .. 3, the same for every chunk
        auto pick = [&](auto shc) {
          constexpr int S = decltype(shc)::value;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            unsigned wd = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int b = 4 * d + e;
              const int pos = b + S;  // float position in the window v[0..4]
              const int code = b0 + b;
              const bool in = code >= 0 && code < rowb;
              const unsigned u = in ? static_cast<unsigned>(static_cast<int32_t>(v[pos >> 2][pos & 3])) - kOff : pad;
              bad |= (u + 128u) > 255u;
              wd |= (u & 0xffu) << (8 * e);
            }
            word[d] = wd;
          }
        };
        switch (sh) {
          case 0: pick(std::integral_constant<int, 0>{}); break;
          case 1: pick(std::integral_constant<int, 1>{}); break;
          case 2: pick(std::integral_constant<int, 2>{}); break;
          default: pick(std::integral_constant<int, 3>{}); break;
        }
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          unsigned wd = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int code = b0 + 4 * d + e;
            const bool in = row_ok && code >= 0 && code < rowb;
            const unsigned u = in ? static_cast<unsigned>(static_cast<int32_t>(src[code])) - kOff : pad;
            bad |= (u + 128u) > 255u;
            wd |= (u & 0xffu) << (8 * e);
          }
          word[d] = wd;
        }
      }
      const v4i o = {static_cast<int>(word[0]), static_cast<int>(word[1]), static_cast<int>(word[2]),
                     static_cast<int>(word[3])};
      *reinterpret_cast<v4i*>(a.xp + idx * 16) = o;
      store_gap(o);
    }
  }
  const int any = __syncthreads_or(bad ? 1 : 0);
  if (t == 0) a.flags[blockIdx.x] = any ? 1 : 0;
}

struct RouteLayout {
  Geom gp;  // the padded problem the stream kernel runs
  size_t xp_off, wq_off, t_off, q_off, f_off, bytes;
  int nfb, nib;
};

size_t rt_align(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

RouteLayout route_layout(const Geom& g) {
  RouteLayout L;
  L.gp = g;
  L.gp.H = g.H + 2 * g.ph;
  L.gp.W = g.W + 2 * g.pw;
  L.gp.ph = 0;
  L.gp.pw = 0;
  const long long kdim = static_cast<long long>(g.R) * g.S * g.Cg;
  const long long nchunks = static_cast<long long>(g.N) * L.gp.H * L.gp.W * (g.C / 16);
  L.nfb = (g.K + 7) / 8;
  L.nib = static_cast<int>((nchunks + kRtThreads - 1) / kRtThreads);
  L.xp_off = 0;
  L.wq_off = rt_align(static_cast<size_t>(nchunks) * 16);
  L.t_off = rt_align(L.wq_off + static_cast<size_t>(g.K) * kdim);
  L.q_off = rt_align(L.t_off + static_cast<size_t>(g.K) * 4);
  L.f_off = rt_align(L.q_off + static_cast<size_t>(g.N) * 16);
  L.bytes = rt_align(L.f_off + static_cast<size_t>(L.nfb + L.nib) * 4);
  return L;
}

bool rt_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct StemLayout {
  Geom gp;  // the padded problem the s2d kernel runs: rows of Wq pixels, no padding, the same Ho, Wo
  size_t xp_off, wq_off, t_off, q_off, f_off, bytes;
  int nfb, nib, cpr;
  long long nchunks;
};

StemLayout stem_layout(const Geom& g) {
  StemLayout L;
  L.gp = g;
  L.gp.H = g.H + 2 * g.ph;
  int wq = g.W + 2 * g.pw;
  while ((static_cast<long long>(wq) * g.C) % 16 != 0) ++wq;
  L.gp.W = wq;
  L.gp.ph = 0;
  L.gp.pw = 0;
  L.cpr = static_cast<int>(static_cast<long long>(wq) * g.C / 16);
  L.nchunks = static_cast<long long>(g.N) * L.gp.H * L.cpr;
  const long long kdim = static_cast<long long>(g.R) * g.S * g.C;
  L.nfb = (g.K + 3) / 4;
  L.nib = static_cast<int>((L.nchunks + kRtThreads - 1) / kRtThreads);  // a 16-byte chunk per thread
  L.xp_off = 0;
  L.wq_off = rt_align(static_cast<size_t>(L.nchunks) * 16);
  L.t_off = rt_align(L.wq_off + static_cast<size_t>(g.K) * kdim);
  L.q_off = rt_align(L.t_off + static_cast<size_t>(g.K) * 4);
  L.f_off = rt_align(L.q_off + static_cast<size_t>(g.N) * 16);
  L.bytes = rt_align(L.f_off + static_cast<size_t>(L.nfb + L.nib) * 4);
  return L;
}

}  // namespace

bool qi32_route_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, const void* y,
                         std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (bg.By != 1 || bg.Bx != 1) return no("qi32 stream route takes plain filters only");
  if (!rt_aligned16(x) || !rt_aligned16(w) || !rt_aligned16(y)) return no("qi32 stream route needs 16-byte aligned x, w and y");
  if (g.C % 16 != 0 || g.H < 1 || g.W < 1) return no("qi32 stream route needs c % 16 == 0 and a non-empty image");
  const RouteLayout L = route_layout(g);
  if (static_cast<long long>(g.N) * L.gp.H * L.gp.W * (g.C / 16) >= (1LL << 31) - kRtThreads) {
    return no("qi32 stream route: padded input too large");
  }
  if (static_cast<long long>(g.N) * g.H * g.W * g.C >= (1LL << 40)) return no("qi32 stream route: input too large");
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  const Requant rq{reinterpret_cast<const int32_t*>(kAligned), reinterpret_cast<const float*>(kAligned), 1.0f, 0};
  return stream_eligible(L.gp, kAligned, kAligned, y, rq, kEpiQi32, why);
}

size_t qi32_route_workspace_bytes(const Geom& g) { return route_layout(g).bytes; }

hipError_t launch_qi32_route(const Geom& g, QpKind qp, const float* x, const float* w, int32_t* y, const void* in_qp,
                             const void* f_qp, void* ws, hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  const RouteLayout L = route_layout(g);
  char* base = static_cast<char*>(ws);
  RoutePrepArgs pa;
  pa.x = x; pa.w = w;
  pa.in_qp = static_cast<const unsigned char*>(in_qp);
  pa.f_qp = static_cast<const unsigned char*>(f_qp);
  pa.xp = reinterpret_cast<int8_t*>(base + L.xp_off);
  pa.wq = reinterpret_cast<int8_t*>(base + L.wq_off);
  pa.T = reinterpret_cast<int32_t*>(base + L.t_off);
  pa.qrec = reinterpret_cast<int32_t*>(base + L.q_off);
  pa.flags = reinterpret_cast<int32_t*>(base + L.f_off);
  pa.N = g.N; pa.H = g.H; pa.W = g.W; pa.C = g.C; pa.K = g.K; pa.Kdim = g.R * g.S * g.Cg;
  pa.ph = g.ph; pa.pw = g.pw; pa.Hp = L.gp.H; pa.Wp = L.gp.W;
  pa.nfb = L.nfb;
  pa.nchunks = static_cast<long long>(g.N) * L.gp.H * L.gp.W * (g.C / 16);
  const dim3 pgrid(static_cast<unsigned>(L.nfb + L.nib));
  if (qp == kQpU8) {
    hipLaunchKernelGGL(qi32_route_prep_kernel<kQpU8>, pgrid, dim3(kRtThreads), 0, stream, pa);
  } else {
    hipLaunchKernelGGL(qi32_route_prep_kernel<kQpS5>, pgrid, dim3(kRtThreads), 0, stream, pa);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_i8_stream_qi32(L.gp, pa.xp, pa.wq, pa.T, pa.qrec, y, stream);
  if (e != hipSuccess) return e;
  RouteFallbackArgs fa;
  fa.x = x; fa.w = w; fa.y = y;
  fa.in_qp = pa.in_qp; fa.f_qp = pa.f_qp;
  fa.flags = pa.flags;
  fa.nflags = L.nfb + L.nib;
  fa.g = g;
  fa.total = static_cast<long long>(g.N) * g.Ho * g.Wo * g.K;
  if (qp == kQpU8) {
    hipLaunchKernelGGL(qi32_route_fallback_kernel<kQpU8>, dim3(256), dim3(kRtThreads), 0, stream, fa);
  } else {
    hipLaunchKernelGGL(qi32_route_fallback_kernel<kQpS5>, dim3(256), dim3(kRtThreads), 0, stream, fa);
  }
  return hipGetLastError();
}

bool qi32_stem_route_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, const void* y,
                              std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (bg.By != 1 || bg.Bx != 1) return no("qi32 stem route takes plain filters only");
  if (!rt_aligned16(x) || !rt_aligned16(w) || !rt_aligned16(y)) return no("qi32 stem route needs 16-byte aligned x, w and y");
  if (g.G != 1 || g.C < 1 || g.C > 4 || g.H < 1 || g.W < 1) {
    return no("qi32 stem route needs groups == 1, 1 <= c <= 4 and a non-empty image");
  }
  if (g.ph < 0 || g.pw < 0) return no("qi32 stem route needs padding >= 0");
  const StemLayout L = stem_layout(g);
  if (L.nchunks >= (1LL << 31) - kRtThreads || static_cast<long long>(g.N) * L.gp.H >= (1LL << 31) - 4) {
    return no("qi32 stem route: padded input too large");
  }
  if (static_cast<long long>(g.N) * g.H * g.W * g.C >= (1LL << 40)) return no("qi32 stem route: input too large");
  return stem_s2d_qi32_plan_ok(L.gp, why);
}

size_t qi32_stem_route_workspace_bytes(const Geom& g) { return stem_layout(g).bytes; }

hipError_t launch_qi32_stem_route(const Geom& g, QpKind qp, const float* x, const float* w, int32_t* y,
                                  const void* in_qp, const void* f_qp, void* ws, hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  const StemLayout L = stem_layout(g);
  char* base = static_cast<char*>(ws);
  StemPrepArgs pa;
  pa.x = x; pa.w = w;
  pa.in_qp = static_cast<const unsigned char*>(in_qp);
  pa.f_qp = static_cast<const unsigned char*>(f_qp);
  pa.xp = reinterpret_cast<int8_t*>(base + L.xp_off);
  pa.wq = reinterpret_cast<int8_t*>(base + L.wq_off);
  pa.T = reinterpret_cast<int32_t*>(base + L.t_off);
  pa.qrec = reinterpret_cast<int32_t*>(base + L.q_off);
  pa.flags = reinterpret_cast<int32_t*>(base + L.f_off);
  pa.N = g.N; pa.H = g.H; pa.W = g.W; pa.C = g.C; pa.K = g.K; pa.Kdim = g.R * g.S * g.C;
  pa.ph = g.ph; pa.pw = g.pw; pa.Hp = L.gp.H; pa.cpr = L.cpr;
  pa.nfb = L.nfb;
  pa.nchunks = L.nchunks;
  const dim3 pgrid(static_cast<unsigned>(L.nfb + L.nib));
  if (qp == kQpU8) {
    hipLaunchKernelGGL(qi32_stem_prep_kernel<kQpU8>, pgrid, dim3(kRtThreads), 0, stream, pa);
  } else {
    hipLaunchKernelGGL(qi32_stem_prep_kernel<kQpS5>, pgrid, dim3(kRtThreads), 0, stream, pa);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_stem_s2d_qi32(L.gp, pa.xp, pa.wq, pa.T, pa.qrec, y, stream);
  if (e != hipSuccess) return e;
  RouteFallbackArgs fa;
  fa.x = x; fa.w = w; fa.y = y;
  fa.in_qp = pa.in_qp; fa.f_qp = pa.f_qp;
  fa.flags = pa.flags;
  fa.nflags = L.nfb + L.nib;
  fa.g = g;
  fa.total = static_cast<long long>(g.N) * g.Ho * g.Wo * g.K;
  if (qp == kQpU8) {
    hipLaunchKernelGGL(qi32_route_fallback_kernel<kQpU8>, dim3(256), dim3(kRtThreads), 0, stream, fa);
  } else {
    hipLaunchKernelGGL(qi32_route_fallback_kernel<kQpS5>, dim3(256), dim3(kRtThreads), 0, stream, fa);
  }
  return hipGetLastError();
}

}  // namespace miq
