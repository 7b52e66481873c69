// int32-accumulator convolution on quantized float codes on the int8 matrix cores: the
// reference's launch_fprop_nhwc_qi32<Tin> (/root/reference/src/conv_types.h:308-323 ->
// cuda_kernels.cu:1336-1392, im2col -> pack -> bmm_matmul_i32 -> unpack), exact for every
// input the reference's CPU definition takes (cpu_ref.cpp:36-72):
//   y[n,ho,wo,g*Kg+ko] = sum over in-bounds taps of (int32(x) - zp_x[n]) * (int32(w) - zp_w)
// with int32 wrap-around, int32() truncating toward zero.
//
// qi32_igemm_kernel: an implicit GEMM whose staging is that of the fp32 implicit GEMM (rows:
// output pixels and one group's output channels; reduction over (r, s, ci) in chunks of 16,
// gathered as float4 of 4 channels of one tap where C/groups % 4 == 0, else value by value) and
// whose arithmetic is that
// of the int32 batched GEMM: every centred code is split into balanced base-256 digits
// (w = (u + 0x808080) ^ 0x808080), and four shift groups of v_mfma_i32_16x16x64_i8 over the
// digit bytes (the filter's byte-reversed and shifted) give the exact wrapped sums.
//   - A workgroup of 8 waves computes 128 pixels x 64 channels; each wave 32 x 32.
//   - Two chunks are in flight per thread on one straight code path: out-of-image taps, values
//     past kdim and rows past M or Kg read a valid address and are zeroed at staging (zero's
//     digits are zero) or never stored.
//   - Per-sample zero points are read once per thread (its pixel's sample); the filter's once.
//   - Blocked filters [K, By, Bx, R, S, C/groups] (launch_block_fprop_nhwc_qi32,
//     cuda_kernels.cu:1394-1461): a workgroup's pixel tile lies inside one filter block of
//     bho x bwo output positions (over the batch), and its filter operand is that block's
//     slice; a plain filter is the case By = Bx = 1.

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kQWaves = 8;
constexpr int kQBM = 128;
constexpr int kQBN = 64;
constexpr int kQKC = 16;
constexpr int kQDepth = 2;

typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

struct Qi32Args {
  const float* x;
  const float* w;
  int32_t* y;
  const unsigned char* in_qp;
  const unsigned char* f_qp;
  Geom g;
  int M, kdim, nchunks, tn, tiles;
  // filter blocks (By = Bx = 1: a plain KRSC filter): a workgroup's pixels lie in one block of
  // bho x bwo output positions; M counts the pixels of one block over the batch
  int By, Bx, bho, bwo, gt;  // gt = tiles * By * Bx
  FastDivM fd_tn, fd_tiles, fd_gt;
};

// Per-sample zero point from the raw parameter struct: uint8 at offset 0 of a 12-byte struct
// (LinQuantU8), int8 at offset 0 of an 8-byte struct (LinQuantS5).
template <QpKind Q>
__device__ __forceinline__ int qp_zero_point(const unsigned char* qp, int i) {
  if constexpr (Q == kQpU8) {
    return static_cast<int>(qp[static_cast<size_t>(i) * 12]);
  } else {
    return static_cast<int>(static_cast<signed char>(qp[static_cast<size_t>(i) * 8]));
  }
}

__device__ __forceinline__ unsigned centred_digits(float code, int zp) {
  const unsigned u = static_cast<unsigned>(static_cast<int32_t>(code) - zp);  // int32 wrap-around
  return (u + 0x808080u) ^ 0x808080u;
}

__device__ __forceinline__ int q_slot(int row, int g) { return 4 * row + (g ^ (((row >> 3) & 1) << 1)); }

struct QTapCursor {
  int r, s, ci;
  __device__ __forceinline__ void step(int Cg, int S) {
    if (++ci == Cg) {
      ci = 0;
      if (++s == S) {
        s = 0;
        ++r;
      }
    }
  }
  __device__ __forceinline__ void advance(int Cg, int S) {
    ci += kQKC;
    while (ci >= Cg) {
      ci -= Cg;
      if (++s == S) {
        s = 0;
        ++r;
      }
    }
  }
};

// V4: a thread's 4 reduction values are 4 channels of one tap, read as one float4 (C/groups % 4
// == 0, 16-byte aligned codes); otherwise each value has its own tap and validity and is read
// alone (any C/groups, e.g. the 3-channel stem), as are the filter's two.
template <QpKind Q, bool V4>
__global__ void __launch_bounds__(64 * kQWaves) __attribute__((amdgpu_waves_per_eu(4, 4))) qi32_igemm_kernel(Qi32Args a) {
  __shared__ v4i sA[2][kQBM * 4];
  __shared__ v4i sB[2][kQBN * 4];
  const Geom& g = a.g;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  const int lin = blockIdx.x;
  const int grp = fdiv(lin, a.fd_gt);
  const int remg = lin - grp * a.gt;
  const int blk = fdiv(remg, a.fd_tiles);
  const int rem = remg - blk * a.tiles;
  const int tmi = fdiv(rem, a.fd_tn);
  const int tni = rem - tmi * a.tn;
  const int bby = blk / a.Bx;
  const int bbx = blk - bby * a.Bx;
  const int m0 = tmi * kQBM;
  const int n0 = tni * kQBN;

  // A: pixel row ar, reduction values 4 aq .. 4 aq + 3 of each chunk
  const int ar = t >> 2;
  const int aq = t & 3;
  const int pix = min(m0 + ar, a.M - 1);
  const int hw = a.bho * a.bwo;
  const int pn = pix / hw;
  const int prem = pix - pn * hw;
  const int pho = bby * a.bho + prem / a.bwo;
  const int pwo = bbx * a.bwo + (prem - (prem / a.bwo) * a.bwo);
  const int hbase = pho * g.sh - g.ph;
  const int wbase = pwo * g.sw - g.pw;
  const float* xn = a.x + static_cast<size_t>(pn) * g.H * g.W * g.C + static_cast<size_t>(grp) * g.Cg;
  const int zx = qp_zero_point<Q>(a.in_qp, pn);
  const int zw = qp_zero_point<Q>(a.f_qp, 0);
  QTapCursor cur;
  {
    const int k = 4 * aq;
    const int tap = k / g.Cg;
    cur.ci = k - tap * g.Cg;
    cur.r = tap / g.S;
    cur.s = tap - cur.r * g.S;
  }
  int cur_chunk = 0;
  // B: filter row br, reduction values 2 bp, 2 bp + 1 of each chunk
  const int br = t >> 3;
  const int bp = t & 7;
  const int brow = grp * g.Kg + min(n0 + br, g.Kg - 1);
  const float* wr = a.w + ((static_cast<size_t>(brow) * a.By + bby) * a.Bx + bbx) * a.kdim;

  // oka / okb: validity bits of the 4 / 2 values (V4: all four share one bit)
  auto load = [&](int c, v4f& va, v2f& vb, unsigned& oka, unsigned& okb) {
    if (cur_chunk < c) {  // chunks are loaded in order; a repeat of the last one does not advance
      cur.advance(g.Cg, g.S);
      ++cur_chunk;
    }
    if constexpr (V4) {
      const int hi = hbase + cur.r * g.dh;
      const int wi = wbase + cur.s * g.dw;
      const bool ok = cur.r < g.R && hi >= 0 && hi < g.H && wi >= 0 && wi < g.W;
      oka = ok ? 0xFu : 0u;
      const size_t xo = ok ? (static_cast<size_t>(hi) * g.W + wi) * g.C + cur.ci : 0;
      va = *reinterpret_cast<const v4f*>(xn + xo);
    } else {
      QTapCursor q = cur;
      oka = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e > 0) q.step(g.Cg, g.S);
        const int hi = hbase + q.r * g.dh;
        const int wi = wbase + q.s * g.dw;
        const bool ok = q.r < g.R && hi >= 0 && hi < g.H && wi >= 0 && wi < g.W;
        oka |= static_cast<unsigned>(ok) << e;
        va[e] = xn[ok ? (static_cast<size_t>(hi) * g.W + wi) * g.C + q.ci : 0];
      }
    }
    const int kb = c * kQKC + 2 * bp;
    if constexpr (V4) {
      okb = kb < a.kdim ? 3u : 0u;
      vb = *reinterpret_cast<const v2f*>(wr + (kb < a.kdim ? kb : 0));
    } else {
      okb = static_cast<unsigned>(kb < a.kdim) | (static_cast<unsigned>(kb + 1 < a.kdim) << 1);
      vb = v2f{wr[(okb & 1u) ? kb : 0], wr[(okb & 2u) ? kb + 1 : 0]};
    }
  };
  const int sa_slot = q_slot(ar, aq);
  const int sb_slot = q_slot(br, bp >> 1);
  auto stage = [&](int buf, const v4f& va, const v2f& vb, unsigned oka, unsigned okb) {
    v4i da;
#pragma unroll
    for (int e = 0; e < 4; ++e) da[e] = ((oka >> e) & 1u) ? static_cast<int>(centred_digits(va[e], zx)) : 0;
    sA[buf][sa_slot] = da;
    v2i db;
#pragma unroll
    for (int e = 0; e < 2; ++e)
      db[e] = ((okb >> e) & 1u) ? static_cast<int>(__builtin_bswap32(centred_digits(vb[e], zw))) : 0;
    *(reinterpret_cast<v2i*>(&sB[buf][sb_slot]) + (bp & 1)) = db;
  };

  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int fb0 = q_slot(32 * wn + (lane & 15), lane >> 4);
  const int fb1 = q_slot(32 * wn + 16 + (lane & 15), lane >> 4);
  const int fa0 = q_slot(32 * wm + (lane & 15), lane >> 4);
  const int fa1 = q_slot(32 * wm + 16 + (lane & 15), lane >> 4);
  v4i acc[4][2][2];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int jn = 0; jn < 2; ++jn)
#pragma unroll
      for (int im = 0; im < 2; ++im) acc[s][jn][im] = v4i{0, 0, 0, 0};

  constexpr int P = kQDepth;
  const int nch = a.nchunks;
  if (nch > 0) {
    const int last = nch - 1;
    v4f va[P];
    v2f vb[P];
    unsigned oka[P], okb[P];
#pragma unroll
    for (int j = 0; j < P; ++j) load(min(j, last), va[j], vb[j], oka[j], okb[j]);
    stage(0, va[0], vb[0], oka[0], okb[0]);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // whole groups of P chunks; chunks past the last load the last one again and stage zeros
    for (int c0 = 0; c0 < nch; c0 += P) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int c = c0 + j;
        load(min(c + P, last), va[j], vb[j], oka[j], okb[j]);  // set j was staged last pass
        const int buf = c & 1;
        const v4i Bf[2] = {sB[buf][fb0], sB[buf][fb1]};
        const v4i Af[2] = {sA[buf][fa0], sA[buf][fa1]};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
          for (int jn = 0; jn < 2; ++jn) {
            const v4i bs = (v4i)((v4u)Bf[jn] >> (8u * static_cast<unsigned>(3 - s)));
#pragma unroll
            for (int im = 0; im < 2; ++im)
              acc[s][jn][im] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bs, Af[im], acc[s][jn][im], 0, 0, 0);
          }
        }
        const int j1 = (j + 1) % P;
        const bool live = c + 1 <= last;
        stage(buf ^ 1, va[j1], vb[j1], live ? oka[j1] : 0u, live ? okb[j1] : 0u);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
    }
  }

  // lane (c = lane % 16, q = lane / 16) of tile (jn, im): pixel m0 + 32 wm + 16 im + c,
  // channels n0 + 32 wn + 16 jn + 4 q .. + 3 of the group
  const bool vec = (g.K & 3) == 0 && (g.Kg & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0;
#pragma unroll
  for (int jn = 0; jn < 2; ++jn) {
#pragma unroll
    for (int im = 0; im < 2; ++im) {
      const int m = m0 + 32 * wm + 16 * im + (lane & 15);
      const int ch = n0 + 32 * wn + 16 * jn + 4 * (lane >> 4);
      v4i r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned v = static_cast<unsigned>(acc[0][jn][im][i]) + (static_cast<unsigned>(acc[1][jn][im][i]) << 8) +
                           (static_cast<unsigned>(acc[2][jn][im][i]) << 16) +
                           (static_cast<unsigned>(acc[3][jn][im][i]) << 24);
        r[i] = static_cast<int>(v);
      }
      if (m >= a.M) continue;
      const int mn = m / hw;
      const int mr = m - mn * hw;
      const int mh = mr / a.bwo;
      const size_t opix = (static_cast<size_t>(mn) * g.Ho + bby * a.bho + mh) * g.Wo + bbx * a.bwo + (mr - mh * a.bwo);
      int32_t* yp = a.y + opix * g.K + static_cast<size_t>(grp) * g.Kg + ch;
      if (vec && ch + 3 < g.Kg) {
        *reinterpret_cast<v4i*>(yp) = r;
        store_gap(r);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (ch + i < g.Kg) yp[i] = r[i];
      }
    }
  }
}

}  // namespace

bool qi32_igemm_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (g.H == 0 || g.W == 0 || g.Cg == 0) return no("qi32 implicit GEMM needs a non-empty input image");
  if ((reinterpret_cast<uintptr_t>(x) & 3u) != 0 || (reinterpret_cast<uintptr_t>(w) & 3u) != 0) {
    return no("qi32 implicit GEMM needs 4-byte aligned x and w");
  }
  const long long m = static_cast<long long>(g.N) * g.Ho * g.Wo;
  const long long kdim = static_cast<long long>(g.R) * g.S * g.Cg;
  if (m >= (1LL << 31) - kQBM || kdim >= (1LL << 31) - kQKC) return no("qi32 implicit GEMM extents exceed int32");
  const long long mb = static_cast<long long>(g.N) * bg.bho * bg.bwo;
  const long long tiles = ((mb + kQBM - 1) / kQBM) * ((g.Kg + kQBN - 1) / kQBN) * g.G * bg.By * bg.Bx;
  if (tiles > (1LL << 22)) return no("qi32 implicit GEMM grid exceeds 2^22 workgroups");
  return true;
}

hipError_t launch_qi32_igemm(const Geom& g, const BlockGeom& bg, QpKind qp, const float* x, const float* w, int32_t* y,
                             const void* in_qp, const void* f_qp, hipStream_t stream) {
  Qi32Args a;
  a.x = x; a.w = w; a.y = y; a.g = g;
  a.in_qp = static_cast<const unsigned char*>(in_qp);
  a.f_qp = static_cast<const unsigned char*>(f_qp);
  a.By = bg.By; a.Bx = bg.Bx; a.bho = bg.bho; a.bwo = bg.bwo;
  a.M = g.N * bg.bho * bg.bwo;
  a.kdim = g.R * g.S * g.Cg;
  a.nchunks = (a.kdim + kQKC - 1) / kQKC;
  a.tn = (g.Kg + kQBN - 1) / kQBN;
  a.tiles = ((a.M + kQBM - 1) / kQBM) * a.tn;
  a.gt = a.tiles * bg.By * bg.Bx;
  a.fd_tn = fastdiv_m(a.tn);
  a.fd_tiles = fastdiv_m(a.tiles);
  a.fd_gt = fastdiv_m(a.gt);
  const unsigned blocks = static_cast<unsigned>(a.gt) * static_cast<unsigned>(g.G);
  const bool v4 = g.Cg % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
  const dim3 grid(blocks), block(64 * kQWaves);
  if (qp == kQpU8) {
    if (v4) hipLaunchKernelGGL((qi32_igemm_kernel<kQpU8, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((qi32_igemm_kernel<kQpU8, false>), grid, block, 0, stream, a);
  } else {
    if (v4) hipLaunchKernelGGL((qi32_igemm_kernel<kQpS5, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((qi32_igemm_kernel<kQpS5, false>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace miq
