// fp32 NHWC convolution, the semantics of the reference's launch_fprop_nhwc
// (/root/reference/src/cuda_kernels.cu:767-823; CPU definition cpu_ref.cpp:116-146):
//   y[n,ho,wo,g*Kg+ko] = sum over in-bounds taps (r, s) and ci < Cg of
//                        x[n, ho*sh-ph+r*dh, wo*sw-pw+s*dw, g*Cg+ci] * w[g*Kg+ko, r, s, ci]
//
// f32_igemm_kernel: implicit GEMM on v_mfma_f32_16x16x4f32.  GEMM rows are output pixels
// (M = N*Ho*Wo) and output channels of one group (Kg); the reduction runs over
// kdim = R*S*Cg in the reference's (r, s, ci) order, in chunks of 16 values.
//   - A workgroup of 8 waves computes 128 pixels x 64 channels of one group; wave w computes
//     channels 32 (w % 2) .. +31 of pixels 32 (w / 2) .. +31: 2 x 2 MFMA tiles.
//   - Staging: each thread gathers one float4 of 4 consecutive input channels of one tap
//     for one pixel (Cg % 4 == 0) and one float2 of its filter row (KRSC rows are
//     kdim-contiguous), into a double-buffered LDS tile [row][16 values] of 64-byte rows
//     whose 16-byte slot g sits at g ^ (2 * bit 3 of the row): a fragment read (16 rows,
//     one slot per lane group) is free of bank conflicts.
//   - A lane's fragment slot holds 4 consecutive reduction values, one per K-step of the
//     chunk's four MFMAs.  The MFMA's A operand is the channel rows, so a lane's
//     accumulators hold 4 consecutive channels of one pixel: one 16-byte NHWC store.
//   - Two chunks are in flight per thread.  Every pass of the loop issues the same loads:
//     taps outside the image, values past kdim and rows past M or Kg read a valid address
//     and are zeroed (or never stored), so the compiler's load counters stay exact.
//   The sum order differs from the reference's sequential fp32 loop; results agree within
//   the reference's own check (verify_tensors with abs 1e-4 / rel 1e-3, main.cpp:306-316).
//
// f32_direct_kernel: one thread per output element, the reference CPU loop order and one
// fp32 multiply and one add per tap (no contraction): the reference CPU result bit for bit.
// Used for every shape the implicit GEMM does not take (Cg % 4 != 0, depthwise, unaligned).
//
// f32_bprop_direct_kernel / f32_grad_direct_kernel: dx and dw (launch_bprop_nhwc,
// launch_grad_nhwc, cuda_kernels.cu:825-937) the same way, in the loop orders of
// cpu_bprop_nhwc / cpu_grad_nhwc: their results bit for bit.

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kF32Waves = 8;
constexpr int kF32BM = 128;  // pixels per workgroup
constexpr int kF32BN = 64;   // channels per workgroup
constexpr int kF32KC = 16;   // reduction values per chunk
constexpr int kF32Depth = 2; // chunks in flight per thread

typedef float v2f __attribute__((ext_vector_type(2)));

struct F32Args {
  const float* x;
  const float* w;
  float* y;
  const float* bias;  // forward with a blocked filter: K * By * Bx floats, or nullptr
  Geom g;
  int M;         // pixel slots per region: N * rh * rw (the pixel-tile grid's extent)
  int kdim;      // R * S * Cg
  int nchunks;   // ceil(kdim / 16)
  int tn;        // channel tiles per group
  int tiles;     // pixel tiles * channel tiles per region
  int ow_taps;   // transposed filter: R * S of the original filter
  int ow_cg;     // transposed filter: channels per group of the original filter (= Kg of g)
  // Output regions: the output grid splits into ry x rx regions of rh x rw positions, the last
  // row and column of regions clipped to Ho x Wo; a workgroup's pixels lie in one region.
  int ry, rx, rh, rw;
  // Filter blocks, By x Bx of bho x bwo positions each (1 x 1 of Ho x Wo: a plain KRSC filter).
  // Forward: the blocks are the regions and a region's pixels use its block's filter.
  // Transposed: the blocks partition this kernel's input (dy), and each input position uses
  // the filter of its block.
  int By, Bx, bho, bwo;
  int bias_mode;  // 0: bias[k][by][bx]; 1: bias[k][0][0] for every block
  int nfast;      // region pixels in (row, column, image) order instead of (image, row, column)
  FastDivM fd_tn, fd_tiles, fd_regions, fd_rx;
};

enum F32Mode : int { kFwd = 0, kTrans = 1, kTransBlocked = 2 };

__device__ __forceinline__ int f32_slot(int row, int g) { return 4 * row + (g ^ (((row >> 3) & 1) << 1)); }

// Gather cursor of one thread's input float4: reduction index k = 16 * chunk + ka, decoded
// as (r, s, ci) and advanced one chunk at a time.
struct TapCursor {
  int r, s, ci;
  __device__ __forceinline__ void advance(int Cg, int S) {
    ci += kF32KC;
    while (ci >= Cg) {
      ci -= Cg;
      if (++s == S) {
        s = 0;
        ++r;
      }
    }
  }
  // the same over taps whose s lies in s0..s1
  __device__ __forceinline__ void advance_in(int Cg, int s0, int s1) {
    ci += kF32KC;
    while (ci >= Cg) {
      ci -= Cg;
      if (++s > s1) {
        s = s0;
        ++r;
      }
    }
  }
};

// floor(a / d) and ceil(a / d) for d > 0 and any sign of a
__device__ __forceinline__ int floor_div(int a, int d) { return a >= 0 ? a / d : -((-a + d - 1) / d); }
__device__ __forceinline__ int ceil_div(int a, int d) { return -floor_div(-a, d); }

// MODE kFwd: the forward convolution (a blocked filter: one block per region).
// MODE kTrans / kTransBlocked (TRANSPOSED): the filter operand is read as the bprop filter of a
// stride-1 convolution:
// row j (an input channel of the original) and reduction index (r', s', ko) address
// w[g Kg + ko][by][bx][R-1-r'][S-1-s'][j] of the original filter (`ow_*` extents in F32Args),
// (by, bx) the block of the input position the tap reads.  kTrans: a plain filter (one block).
// kTransBlocked: a workgroup runs its reduction once per filter block that its pixels' taps can
// reach, over the taps that reach it, reading only the input positions of that block each time.
// BN: channels per workgroup, 64 (128 pixels, waves 4 x 2) or 32 for groups of at most 32
// output channels (256 pixels, waves 8 x 1; each thread stages two pixel rows, and the waves
// of threads 256.. load filter rows again without staging them).
template <int MODE, int BN>
__global__ void __launch_bounds__(64 * kF32Waves, 1) f32_igemm_kernel(F32Args a) {
  constexpr bool TRANSPOSED = MODE != kFwd;
  constexpr bool MULTI = MODE == kTransBlocked;  // several filter blocks per tile
  constexpr int BM = BN == 64 ? 128 : 256;
  constexpr int NA = BM / 128;  // pixel rows per thread
  __shared__ v4f sA[2][BM * 4];
  __shared__ v4f sB[2][BN * 4];
  const Geom& g = a.g;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  const int lin = blockIdx.x;
  const int gr = fdiv(lin, a.fd_tiles);  // group * regions + region
  const int rem = lin - gr * a.tiles;
  const int grp = fdiv(gr, a.fd_regions);
  const int reg = gr - grp * (a.ry * a.rx);
  const int rgy = fdiv(reg, a.fd_rx);
  const int rgx = reg - rgy * a.rx;
  const int tmi = fdiv(rem, a.fd_tn);
  const int tni = rem - tmi * a.tn;
  const int row0 = rgy * a.rh;
  const int col0 = rgx * a.rw;
  const int rows = min(a.rh, g.Ho - row0);
  const int cols = min(a.rw, g.Wo - col0);
  const int Mr = rows > 0 && cols > 0 ? g.N * rows * cols : 0;  // this region's pixels
  const int rc = rows * cols;
  const int m0 = tmi * BM;
  const int n0 = tni * BN;
  if (m0 >= Mr) return;  // whole workgroup, before any barrier: a tile past a clipped region

  // Region pixel m -> (image, row, column): batch-slowest, or with a.nfast batch-fastest, so that
  // a tile spans few positions and (transposed, blocked filter) reaches few filter blocks.
  auto decode = [&](int m, int& pn, int& lr, int& lc) {
    if (MULTI && a.nfast) {
      const int pos = m / g.N;
      pn = m - pos * g.N;
      lr = pos / cols;
      lc = pos - lr * cols;
    } else {
      pn = m / rc;
      const int prem = m - pn * rc;
      lr = prem / cols;
      lc = prem - lr * cols;
    }
  };

  // A: pixel rows ar + 128 i, reduction values 4 aq .. 4 aq + 3 of each chunk
  const int ar = t >> 2;
  const int aq = t & 3;
  int hbase[NA], wbase[NA];
  const float* xn[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    int pn, lr, lc;
    decode(min(m0 + ar + 128 * i, Mr - 1), pn, lr, lc);
    hbase[i] = (row0 + lr) * g.sh - g.ph;
    wbase[i] = (col0 + lc) * g.sw - g.pw;
    xn[i] = a.x + static_cast<size_t>(pn) * g.H * g.W * g.C + static_cast<size_t>(grp) * g.Cg;
  }
  TapCursor cur;
  {
    const int k = 4 * aq;
    const int tap = k / g.Cg;
    cur.ci = k - tap * g.Cg;
    cur.r = tap / g.S;
    cur.s = tap - cur.r * g.S;
  }
  int cur_chunk = 0;
  // B: filter row br (channel of the group), reduction values 2 bp, 2 bp + 1 of each chunk
  const int br = (t >> 3) & (BN - 1);
  const int bp = t & 7;
  const bool b_stager = BN == 64 || t < 8 * BN;  // whole waves
  const int nblk = a.By * a.Bx;
  const int brow = grp * g.Kg + min(n0 + br, g.Kg - 1);
  const float* wr = a.w + (static_cast<size_t>(brow) * nblk + (TRANSPOSED ? 0 : reg)) * a.kdim;
  // transposed filter: this thread's row is input channel bj of the original filter, its
  // reduction values (r', s', ko), (r', s', ko + 1) of each chunk tracked by a cursor
  const int bj = min(n0 + br, g.Kg - 1);
  const size_t blk_stride = static_cast<size_t>(a.ow_taps) * a.ow_cg;  // between filter blocks
  const size_t ko_stride = blk_stride * nblk;                          // between original channels
  const float* wt0 = a.w + static_cast<size_t>(grp) * g.Cg * ko_stride + bj;  // (ko = 0, block 0, r = s = 0)
  TapCursor bcur{0, 0, 0};
  if constexpr (MODE == kTrans) {
    const int k = 2 * bp;
    const int tap = k / g.Cg;
    bcur.ci = k - tap * g.Cg;
    bcur.r = tap / g.S;
    bcur.s = tap - bcur.r * g.S;
  }

  // Transposed: the filter blocks this tile's taps can reach (inclusive rectangle qy0..qy1 x
  // qx0..qx1), from the tile's range of output rows t_hlo..t_hhi and columns t_wlo..t_whi; a
  // plain filter has the one block 0.  Input rows read by output row y: y sh - ph + r dh.
  int qy0 = 0, qy1 = 0, qx0 = 0, qx1 = 0;
  int nrect = 1;
  int t_hlo = 0, t_hhi = 0, t_wlo = 0, t_whi = 0;
  if constexpr (MULTI) {
    const int p1 = min(m0 + BM, Mr) - 1;
    int rlo = 0, rhi = rows - 1, clo = 0, chi = cols - 1;
    if (a.nfast) {
      const int pos0 = m0 / g.N, pos1 = p1 / g.N;
      rlo = pos0 / cols;
      rhi = pos1 / cols;
      if (rlo == rhi) {
        clo = pos0 - rlo * cols;
        chi = pos1 - rhi * cols;
      }
    } else {
      const int pn0 = m0 / rc, pn1 = p1 / rc;
      const int lr0 = (m0 - pn0 * rc) / cols, lr1 = (p1 - pn1 * rc) / cols;
      if (pn0 == pn1) {
        rlo = lr0;
        rhi = lr1;
        if (lr0 == lr1) {
          clo = m0 - pn0 * rc - lr0 * cols;
          chi = p1 - pn1 * rc - lr1 * cols;
        }
      }
    }
    t_hlo = row0 + rlo;
    t_hhi = row0 + rhi;
    t_wlo = col0 + clo;
    t_whi = col0 + chi;
    const int ylo = max(t_hlo * g.sh - g.ph + min(0, (g.R - 1) * g.dh), 0);
    const int yhi = min(t_hhi * g.sh - g.ph + max(0, (g.R - 1) * g.dh), g.H - 1);
    const int xlo = max(t_wlo * g.sw - g.pw + min(0, (g.S - 1) * g.dw), 0);
    const int xhi = min(t_whi * g.sw - g.pw + max(0, (g.S - 1) * g.dw), g.W - 1);
    if (ylo <= yhi && xlo <= xhi) {
      qy0 = ylo / a.bho;
      qy1 = yhi / a.bho;
      qx0 = xlo / a.bwo;
      qx1 = xhi / a.bwo;
      nrect = (qy1 - qy0 + 1) * (qx1 - qx0 + 1);
    } else {
      nrect = 0;  // no tap reads the input: the tile is zero
    }
  }
  // The taps r0..r1 x s0..s1 that read block (by_, bx_) for some pixel of the tile, and the
  // chunks of that block's reduction (r, s, ko): taps outside read nothing of the block.
  // Non-positive dilation keeps every tap.
  auto block_red = [&](int by_, int bx_, int& r0, int& r1, int& s0, int& s1) -> int {
    const int y0 = by_ * a.bho, y1 = min(y0 + a.bho, g.H) - 1;
    const int x0 = bx_ * a.bwo, x1 = min(x0 + a.bwo, g.W) - 1;
    r0 = 0; r1 = g.R - 1; s0 = 0; s1 = g.S - 1;
    if (g.dh > 0) {
      r0 = max(r0, ceil_div(y0 - t_hhi * g.sh + g.ph, g.dh));
      r1 = min(r1, floor_div(y1 - t_hlo * g.sh + g.ph, g.dh));
    }
    if (g.dw > 0) {
      s0 = max(s0, ceil_div(x0 - t_whi * g.sw + g.pw, g.dw));
      s1 = min(s1, floor_div(x1 - t_wlo * g.sw + g.pw, g.dw));
    }
    if (r0 > r1 || s0 > s1) return 0;
    return ((r1 - r0 + 1) * (s1 - s0 + 1) * g.Cg + kF32KC - 1) / kF32KC;
  };
  int nch = a.nchunks;  // chunks of the whole reduction (one block, every tap)
  if constexpr (MULTI) {
    nch = 0;
    for (int y = qy0; y < qy0 + (nrect > 0 ? qy1 - qy0 + 1 : 0); ++y)
      for (int x = qx0; x <= qx1; ++x) {
        int r0, r1, s0, s1;
        nch += block_red(y, x, r0, r1, s0, s1);
      }
  }
  // current block of the reduction, the input positions it covers and its taps
  int qy = qy0, qx = qx0, cib = 0;
  int ylo_b = 0, yhi_b = g.H, xlo_b = 0, xhi_b = g.W;
  int nch_b = a.nchunks, kd_b = a.kdim, r0b = 0, r1b = g.R - 1, s0b = 0, s1b = g.S - 1;
  const float* wtb = wt0;
  auto set_block = [&]() {
    ylo_b = qy * a.bho;
    yhi_b = min(ylo_b + a.bho, g.H);
    xlo_b = qx * a.bwo;
    xhi_b = min(xlo_b + a.bwo, g.W);
    wtb = wt0 + static_cast<size_t>(qy * a.Bx + qx) * blk_stride;
    nch_b = block_red(qy, qx, r0b, r1b, s0b, s1b);
    kd_b = nch_b > 0 ? (r1b - r0b + 1) * (s1b - s0b + 1) * g.Cg : 0;
  };
  auto start_block = [&]() {  // both cursors at the block's first chunk
    const int ns = s1b - s0b + 1;
    int tap = (4 * aq) / g.Cg;
    cur.ci = 4 * aq - tap * g.Cg;
    cur.r = r0b + tap / ns;
    cur.s = s0b + tap % ns;
    tap = (2 * bp) / g.Cg;
    bcur.ci = 2 * bp - tap * g.Cg;
    bcur.r = r0b + tap / ns;
    bcur.s = s0b + tap % ns;
  };
  auto next_block = [&]() {  // the next block of the rectangle with taps to run
    while (qy <= qy1) {
      if (++qx > qx1) {
        qx = qx0;
        ++qy;
      }
      if (qy > qy1) break;  // not reached: the chunk count covers the live blocks only
      set_block();
      if (nch_b > 0) break;
    }
    start_block();
  };
  if constexpr (MULTI) {
    if (nch > 0) {
      set_block();
      if (nch_b == 0) next_block();
      else start_block();
    }
  }

  auto load = [&](int c, v4f (&va)[NA], v2f& vb, unsigned& oka, bool& okb) {
    if (cur_chunk < c) {  // chunks are loaded in order; a repeat of the last one does not advance
      ++cur_chunk;
      if constexpr (MULTI) {
        if (++cib == nch_b) {  // next block of the tile's rectangle
          cib = 0;
          next_block();
        } else {
          cur.advance_in(g.Cg, s0b, s1b);
          bcur.advance_in(g.Cg, s0b, s1b);
        }
      } else {
        cur.advance(g.Cg, g.S);
        if constexpr (TRANSPOSED) bcur.advance(g.Cg, g.S);
        cib = cur_chunk;
      }
    }
    oka = 0;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int hi = hbase[i] + cur.r * g.dh;
      const int wi = wbase[i] + cur.s * g.dw;
      const bool ok = cur.r <= r1b && hi >= ylo_b && hi < yhi_b && wi >= xlo_b && wi < xhi_b;
      oka |= static_cast<unsigned>(ok) << i;
      const size_t xo = ok ? (static_cast<size_t>(hi) * g.W + wi) * g.C + cur.ci : 0;
      va[i] = *reinterpret_cast<const v4f*>(xn[i] + xo);
    }
    const int kb = cib * kF32KC + 2 * bp;
    okb = kb < kd_b;
    if constexpr (TRANSPOSED) {
      // original filter w[ko][by][bx][R-1-r'][S-1-s'][bj], ko = bcur.ci (+1)
      const size_t tap = static_cast<size_t>(g.R - 1 - bcur.r) * g.S + (g.S - 1 - bcur.s);
      const size_t o = okb ? static_cast<size_t>(bcur.ci) * ko_stride + tap * a.ow_cg : 0;
      vb = v2f{wtb[o], wtb[o + static_cast<size_t>(okb) * ko_stride]};
    } else {
      vb = *reinterpret_cast<const v2f*>(wr + (okb ? kb : 0));
    }
  };
  const int sb_slot = f32_slot(br, bp >> 1);
  auto stage = [&](int buf, const v4f (&va)[NA], const v2f& vb, unsigned oka, bool okb) {
#pragma unroll
    for (int i = 0; i < NA; ++i) sA[buf][f32_slot(ar + 128 * i, aq)] = ((oka >> i) & 1u) ? va[i] : v4f{0.f, 0.f, 0.f, 0.f};
    if (b_stager) *(reinterpret_cast<v2f*>(&sB[buf][sb_slot]) + (bp & 1)) = okb ? vb : v2f{0.f, 0.f};
  };

  const int wn = BN == 64 ? (wave & 1) : 0;
  const int wm = BN == 64 ? (wave >> 1) : wave;
  const int fb0 = f32_slot(32 * wn + (lane & 15), lane >> 4);
  const int fb1 = f32_slot(32 * wn + 16 + (lane & 15), lane >> 4);
  const int fa0 = f32_slot(32 * wm + (lane & 15), lane >> 4);
  const int fa1 = f32_slot(32 * wm + 16 + (lane & 15), lane >> 4);
  v4f acc[2][2];
#pragma unroll
  for (int jn = 0; jn < 2; ++jn)
#pragma unroll
    for (int im = 0; im < 2; ++im) acc[jn][im] = v4f{0.f, 0.f, 0.f, 0.f};

  constexpr int P = kF32Depth;
  if (nch > 0) {
    const int last = nch - 1;
    v4f va[P][NA];
    v2f vb[P];
    unsigned oka[P];
    bool okb[P];
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
        const v4f Bf[2] = {sB[buf][fb0], sB[buf][fb1]};
        const v4f Af[2] = {sA[buf][fa0], sA[buf][fa1]};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int im = 0; im < 2; ++im)
              acc[jn][im] = __builtin_amdgcn_mfma_f32_16x16x4f32(Bf[jn][kk], Af[im][kk], acc[jn][im], 0, 0, 0);
        const int jn1 = (j + 1) % P;
        const bool live = c + 1 <= last;
        stage(buf ^ 1, va[jn1], vb[jn1], live ? oka[jn1] : 0u, live && okb[jn1]);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
    }
  }

  // lane (c = lane % 16, q = lane / 16) of tile (jn, im): pixel m0 + 32 wm + 16 im + c,
  // channels n0 + 32 wn + 16 jn + 4 q .. + 3 of the group
  const bool vec = (g.K & 3) == 0 && (g.Kg & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0;
  const float* bias = TRANSPOSED ? nullptr : a.bias;
  const int bias_y = a.bias_mode == 0 ? rgy : 0;
  const int bias_x = a.bias_mode == 0 ? rgx : 0;
#pragma unroll
  for (int im = 0; im < 2; ++im) {
    const int m = m0 + 32 * wm + 16 * im + (lane & 15);
    if (m >= Mr) continue;
    int pn, lr, lc;
    decode(m, pn, lr, lc);
    const size_t pix = (static_cast<size_t>(pn) * g.Ho + row0 + lr) * g.Wo + col0 + lc;
#pragma unroll
    for (int jn = 0; jn < 2; ++jn) {
      const int ch = n0 + 32 * wn + 16 * jn + 4 * (lane >> 4);
      float* yp = a.y + pix * g.K + static_cast<size_t>(grp) * g.Kg + ch;
      v4f r = acc[jn][im];
      if (bias != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k = grp * g.Kg + min(ch + i, g.Kg - 1);
          r[i] = __fadd_rn(r[i], bias[(static_cast<size_t>(k) * a.By + bias_y) * a.Bx + bias_x]);
        }
      }
      if (vec && ch + 3 < g.Kg) {
        *reinterpret_cast<v4f*>(yp) = r;
        store_gap(r);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (ch + i < g.Kg) yp[i] = r[i];
      }
    }
  }
}

constexpr int kDirectThreads = 256;

// Element index -> (outer..., inner) by three launch-constant divisors; below 2^31 elements
// with the multiply-high division (FastDivM), else in 64-bit arithmetic.
struct Split3 {
  FastDivM d0, d1, d2;  // innermost divisor first
  int v0, v1, v2;
  __device__ __forceinline__ void apply(long long e, bool small, int& i0, int& i1, int& i2, int& i3) const {
    if (small) {
      const int a = static_cast<int>(e);
      const int q0 = fdiv(a, d0);
      i0 = a - q0 * v0;
      const int q1 = fdiv(q0, d1);
      i1 = q0 - q1 * v1;
      i3 = fdiv(q1, d2);
      i2 = q1 - i3 * v2;
    } else {
      i0 = static_cast<int>(e % v0);
      const long long q0 = e / v0;
      i1 = static_cast<int>(q0 % v1);
      const long long q1 = q0 / v1;
      i2 = static_cast<int>(q1 % v2);
      i3 = static_cast<int>(q1 / v2);
    }
  }
};

inline Split3 make_split3(int v0, int v1, int v2) {
  return Split3{fastdiv_m(static_cast<uint32_t>(v0)), fastdiv_m(static_cast<uint32_t>(v1)),
                fastdiv_m(static_cast<uint32_t>(v2)), v0, v1, v2};
}

// With a blocked filter (bg: By x Bx blocks of bho x bwo output positions) the output position
// (ho, wo) takes the filter w[k][ho / bho][wo / bwo] and, after the tap sum, one fp32 add of
// its bias (bias[k][by][bx], or bias[k][0][0] with bias_mode 1), as cpu_block_fprop_nhwc
// (cpu_ref.cpp:232-270) does.
__global__ void __launch_bounds__(kDirectThreads) f32_direct_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ w,
                                                                    float* __restrict__ y, Geom g, BlockGeom bg,
                                                                    const float* __restrict__ bias, int bias_mode,
                                                                    long long total, Split3 sp) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  int k, wo, ho, n;
  sp.apply(e, total < (1LL << 31), k, wo, ho, n);
  const int grp = k / g.Kg;
  const int by = ho / bg.bho, bx = wo / bg.bwo;
  const float* wk = w + (static_cast<size_t>(k) * bg.By * bg.Bx + by * bg.Bx + bx) * g.R * g.S * g.Cg;
  const float* xg = x + static_cast<size_t>(n) * g.H * g.W * g.C + static_cast<size_t>(grp) * g.Cg;
  float acc = 0.0f;
  for (int r = 0; r < g.R; ++r) {
    const int hi = ho * g.sh - g.ph + r * g.dh;
    if (hi < 0 || hi >= g.H) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wi = wo * g.sw - g.pw + s * g.dw;
      if (wi < 0 || wi >= g.W) continue;
      const float* xp = xg + (static_cast<size_t>(hi) * g.W + wi) * g.C;
      const float* wp = wk + (static_cast<size_t>(r) * g.S + s) * g.Cg;
      for (int ci = 0; ci < g.Cg; ++ci) acc = __fadd_rn(acc, __fmul_rn(xp[ci], wp[ci]));
    }
  }
  if (bias != nullptr) {
    acc = __fadd_rn(acc, bias[(static_cast<size_t>(k) * bg.By + (bias_mode == 0 ? by : 0)) * bg.Bx +
                              (bias_mode == 0 ? bx : 0)]);
  }
  y[e] = acc;
}

// Depthwise fp32 convolution (C/groups == K/groups == 1, C % 4 == 0): one thread per output
// pixel and 4 consecutive channels, one float4 of the input per tap; the filter is staged in
// LDS transposed to [tap][channel], so a tap's 4 weights are one 16-byte LDS read.  Each
// channel's sum runs over (r, s) in the reference loop's order with one multiply and one add
// per tap, so the result is cpu_fprop_nhwc's bit for bit.
constexpr int kDwLdsFloats = 8192;  // R * S * C staged per workgroup (32 KB)

__global__ void __launch_bounds__(kDirectThreads) f32_depthwise_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ w,
                                                                       float* __restrict__ y, Geom g, long long total,
                                                                       Split3 sp) {
  __shared__ v4f wl[kDwLdsFloats / 4];
  const int taps = g.R * g.S;
  float* wf = reinterpret_cast<float*>(wl);
  for (int i = threadIdx.x; i < taps * g.C; i += kDirectThreads) {  // w[c][t] -> wl[t][c]
    const int c = i / taps;
    const int t = i - c * taps;
    wf[t * g.C + c] = w[i];
  }
  __syncthreads();
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;  // after the only barrier
  int c4, wo, ho, n;
  sp.apply(e, total < (1LL << 31), c4, wo, ho, n);
  const int c = 4 * c4;
  const float* xn = x + static_cast<size_t>(n) * g.H * g.W * g.C + c;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < g.R; ++r) {
    const int hi = ho * g.sh - g.ph + r * g.dh;
    if (hi < 0 || hi >= g.H) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wi = wo * g.sw - g.pw + s * g.dw;
      if (wi < 0 || wi >= g.W) continue;
      const v4f xv = *reinterpret_cast<const v4f*>(xn + (static_cast<size_t>(hi) * g.W + wi) * g.C);
      const v4f wv = wl[((r * g.S + s) * g.C + c) >> 2];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(xv[j], wv[j]));
    }
  }
  const size_t pix = (static_cast<size_t>(n) * g.Ho + ho) * g.Wo + wo;
  *reinterpret_cast<v4f*>(y + pix * g.K + c) = acc;
  store_gap(acc);
}

// Depthwise fp32 dw (C/groups == K/groups == 1, C % 4 == 0, R*S <= 16): one thread per 4
// channels and a run of kDwGradPix consecutive output pixels, summing x * dy for all R*S taps
// in registers (float4 reads of x and dy).  With `part` the thread stores its partial sums at
// part[run][c][tap] (every entry of every run is written) and f32_sum_parts_kernel adds the
// runs in order: the same result on every call.  Without it they are added into dw (zeroed
// first) with float atomics, whose order varies from run to run.  Either order differs from
// cpu_grad_nhwc's.
constexpr int kDwGradPix = 128;
constexpr int kDwGradTaps = 16;

__global__ void __launch_bounds__(kDirectThreads) f32_depthwise_grad_kernel(const float* __restrict__ x,
                                                                            const float* __restrict__ dy,
                                                                            float* __restrict__ dw,
                                                                            float* __restrict__ part, Geom g, int P,
                                                                            long long total) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  const int c4n = g.C / 4;
  const int c = 4 * static_cast<int>(e % c4n);
  const int p0 = static_cast<int>(e / c4n) * kDwGradPix;
  const int p1 = min(P, p0 + kDwGradPix);
  const int taps = g.R * g.S;
  v4f acc[kDwGradTaps];
#pragma unroll
  for (int t = 0; t < kDwGradTaps; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int hw = g.Ho * g.Wo;
  int n = p0 / hw;
  int ho = (p0 - n * hw) / g.Wo;
  int wo = p0 - n * hw - ho * g.Wo;
  for (int p = p0; p < p1; ++p) {
    const v4f dv = *reinterpret_cast<const v4f*>(dy + static_cast<size_t>(p) * g.K + c);
    const float* xn = x + static_cast<size_t>(n) * g.H * g.W * g.C + c;
#pragma unroll
    for (int t = 0; t < kDwGradTaps; ++t) {
      if (t < taps) {
        const int r = t / g.S;
        const int s = t - r * g.S;
        const int hi = ho * g.sh - g.ph + r * g.dh;
        const int wi = wo * g.sw - g.pw + s * g.dw;
        if (hi >= 0 && hi < g.H && wi >= 0 && wi < g.W) {
          const v4f xv = *reinterpret_cast<const v4f*>(xn + (static_cast<size_t>(hi) * g.W + wi) * g.C);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[t][j] = __fadd_rn(acc[t][j], __fmul_rn(xv[j], dv[j]));
        }
      }
    }
    if (++wo == g.Wo) {
      wo = 0;
      if (++ho == g.Ho) {
        ho = 0;
        ++n;
      }
    }
  }
  if (part != nullptr) {
    float* pr = part + static_cast<size_t>(p0 / kDwGradPix) * g.C * taps;
#pragma unroll
    for (int t = 0; t < kDwGradTaps; ++t)
      if (t < taps)
#pragma unroll
        for (int j = 0; j < 4; ++j) pr[static_cast<size_t>(c + j) * taps + t] = acc[t][j];
    return;
  }
#pragma unroll
  for (int t = 0; t < kDwGradTaps; ++t)
    if (t < taps)
#pragma unroll
      for (int j = 0; j < 4; ++j) unsafeAtomicAdd(dw + static_cast<size_t>(c + j) * taps + t, acc[t][j]);
}

// dw[i] = part[0][i] + part[1][i] + ... + part[nparts - 1][i], in that order (one thread per
// element, `count` elements per part): the deterministic sum of the split partial tiles.
__global__ void __launch_bounds__(kDirectThreads) f32_sum_parts_kernel(const float* __restrict__ part,
                                                                       float* __restrict__ dw, long long count,
                                                                       int nparts) {
  const long long stride = static_cast<long long>(gridDim.x) * kDirectThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x; i < count; i += stride) {
    float acc = part[i];
    for (int s = 1; s < nparts; ++s) acc = __fadd_rn(acc, part[static_cast<size_t>(s) * count + i]);
    dw[i] = acc;
  }
}

// dx of the convolution, the reference's cpu_bprop_nhwc order (cpu_ref.cpp:150-190): one
// thread per dx element; for each tap (r, s) whose output position ho = (hi + ph - r dh) / sh
// is whole and in range (likewise wo), acc += dy * w over the group's output channels.  With a
// blocked filter each tap takes the filter of its output position's block, as
// cpu_block_bprop_nhwc (cpu_ref.cpp:272-314) does.
__global__ void __launch_bounds__(kDirectThreads) f32_bprop_direct_kernel(const float* __restrict__ dy,
                                                                          const float* __restrict__ w,
                                                                          float* __restrict__ dx, Geom g,
                                                                          BlockGeom bg, long long total, Split3 sp) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  int c, wi, hi, n;
  sp.apply(e, total < (1LL << 31), c, wi, hi, n);
  const int grp = c / g.Cg;
  const int ci = c - grp * g.Cg;
  const size_t tstride = static_cast<size_t>(g.R) * g.S * g.Cg;    // between filter blocks
  const size_t wstride = tstride * bg.By * bg.Bx;                 // between output channels
  float acc = 0.0f;
  for (int r = 0; r < g.R; ++r) {
    const int hn = hi + g.ph - r * g.dh;
    if (hn < 0 || hn % g.sh != 0) continue;
    const int ho = hn / g.sh;
    if (ho >= g.Ho) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wn = wi + g.pw - s * g.dw;
      if (wn < 0 || wn % g.sw != 0) continue;
      const int wo = wn / g.sw;
      if (wo >= g.Wo) continue;
      const float* dyp = dy + ((static_cast<size_t>(n) * g.Ho + ho) * g.Wo + wo) * g.K + static_cast<size_t>(grp) * g.Kg;
      const int blk = (ho / bg.bho) * bg.Bx + wo / bg.bwo;
      const float* wp = w + static_cast<size_t>(grp) * g.Kg * wstride + blk * tstride +
                        (static_cast<size_t>(r) * g.S + s) * g.Cg + ci;
      for (int ko = 0; ko < g.Kg; ++ko) acc = __fadd_rn(acc, __fmul_rn(dyp[ko], wp[ko * wstride]));
    }
  }
  dx[e] = acc;
}

// The same dx with 4 consecutive input channels per thread ((C/groups) % 4 == 0, dx and the
// filter 16-byte aligned): per output channel one float4 of the filter (KRSC rows are
// ci-contiguous) and one dy value shared by the 4 sums.  Each channel's sum keeps the (r, s, ko)
// order of cpu_bprop_nhwc with one multiply and one add per term, so dx is the direct kernel's
// bit for bit; the loads per multiply-add drop from 2 to 1/2.
__global__ void __launch_bounds__(kDirectThreads) f32_bprop_direct4_kernel(const float* __restrict__ dy,
                                                                           const float* __restrict__ w,
                                                                           float* __restrict__ dx, Geom g,
                                                                           BlockGeom bg, long long total, Split3 sp) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  int c4, wi, hi, n;
  sp.apply(e, total < (1LL << 31), c4, wi, hi, n);
  const int c = 4 * c4;
  const int grp = c / g.Cg;
  const int ci = c - grp * g.Cg;
  const size_t tstride = static_cast<size_t>(g.R) * g.S * g.Cg;    // between filter blocks
  const size_t wstride = tstride * bg.By * bg.Bx;                 // between output channels
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < g.R; ++r) {
    const int hn = hi + g.ph - r * g.dh;
    if (hn < 0 || hn % g.sh != 0) continue;
    const int ho = hn / g.sh;
    if (ho >= g.Ho) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wn = wi + g.pw - s * g.dw;
      if (wn < 0 || wn % g.sw != 0) continue;
      const int wo = wn / g.sw;
      if (wo >= g.Wo) continue;
      const float* dyp = dy + ((static_cast<size_t>(n) * g.Ho + ho) * g.Wo + wo) * g.K + static_cast<size_t>(grp) * g.Kg;
      const int blk = (ho / bg.bho) * bg.Bx + wo / bg.bwo;
      const float* wp = w + static_cast<size_t>(grp) * g.Kg * wstride + blk * tstride +
                        (static_cast<size_t>(r) * g.S + s) * g.Cg + ci;
      for (int ko = 0; ko < g.Kg; ++ko) {
        const float d = dyp[ko];
        const v4f wv = *reinterpret_cast<const v4f*>(wp + ko * wstride);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(d, wv[j]));
      }
    }
  }
  *reinterpret_cast<v4f*>(dx + 4 * e) = acc;
  store_gap(acc);
}

// Depthwise dx (C/groups == K/groups == 1, C % 4 == 0, plain filter): one thread per input
// pixel and 4 consecutive channels, the filter staged in LDS as [tap][channel] as in
// f32_depthwise_kernel, one float4 of dy per tap.  Channel c's sum runs over the taps (r, s)
// whose output position is whole and in range, in cpu_bprop_nhwc's order with its single
// output channel: dx is the direct kernel's bit for bit, at any stride.
__global__ void __launch_bounds__(kDirectThreads) f32_depthwise_bprop_kernel(const float* __restrict__ dy,
                                                                             const float* __restrict__ w,
                                                                             float* __restrict__ dx, Geom g,
                                                                             long long total, Split3 sp) {
  __shared__ v4f wl[kDwLdsFloats / 4];
  const int taps = g.R * g.S;
  float* wf = reinterpret_cast<float*>(wl);
  for (int i = threadIdx.x; i < taps * g.C; i += kDirectThreads) {  // w[c][t] -> wl[t][c]
    const int c = i / taps;
    const int t = i - c * taps;
    wf[t * g.C + c] = w[i];
  }
  __syncthreads();
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;  // after the only barrier
  int c4, wi, hi, n;
  sp.apply(e, total < (1LL << 31), c4, wi, hi, n);
  const int c = 4 * c4;
  const float* dyn = dy + static_cast<size_t>(n) * g.Ho * g.Wo * g.K + c;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < g.R; ++r) {
    const int hn = hi + g.ph - r * g.dh;
    if (hn < 0 || hn % g.sh != 0) continue;
    const int ho = hn / g.sh;
    if (ho >= g.Ho) continue;
    for (int s = 0; s < g.S; ++s) {
      const int wn = wi + g.pw - s * g.dw;
      if (wn < 0 || wn % g.sw != 0) continue;
      const int wo = wn / g.sw;
      if (wo >= g.Wo) continue;
      const v4f dv = *reinterpret_cast<const v4f*>(dyn + (static_cast<size_t>(ho) * g.Wo + wo) * g.K);
      const v4f wv = wl[((r * g.S + s) * g.C + c) >> 2];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(dv[j], wv[j]));
    }
  }
  *reinterpret_cast<v4f*>(dx + 4 * e) = acc;
  store_gap(acc);
}

// dw of the convolution, the reference's cpu_grad_nhwc order (cpu_ref.cpp:192-230): one thread
// per dw[k][r][s][ci] element, acc += x * dy over n, ho, wo in that order (in-bounds taps).
// With a blocked filter, per dw[k][by][bx][r][s][ci] element over n and the block's positions,
// the order of cpu_block_grad_nhwc (cpu_ref.cpp:316-369).
__global__ void __launch_bounds__(kDirectThreads) f32_grad_direct_kernel(const float* __restrict__ x,
                                                                         const float* __restrict__ dy,
                                                                         float* __restrict__ dw, Geom g,
                                                                         BlockGeom bg, long long total) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  const int ci = static_cast<int>(e % g.Cg);
  const long long t1 = e / g.Cg;
  const int s = static_cast<int>(t1 % g.S);
  const long long t2 = t1 / g.S;
  const int r = static_cast<int>(t2 % g.R);
  const long long t3 = t2 / g.R;
  const int nblk = bg.By * bg.Bx;
  const int blk = static_cast<int>(t3 % nblk);
  const int k = static_cast<int>(t3 / nblk);
  const int ho0 = (blk / bg.Bx) * bg.bho;
  const int wo0 = (blk - (blk / bg.Bx) * bg.Bx) * bg.bwo;
  const int grp = k / g.Kg;
  const float* xc = x + static_cast<size_t>(grp) * g.Cg + ci;
  const float* dyk = dy + k;
  float acc = 0.0f;
  for (int n = 0; n < g.N; ++n) {
    for (int ho = ho0; ho < ho0 + bg.bho; ++ho) {
      const int hi = ho * g.sh - g.ph + r * g.dh;
      if (hi < 0 || hi >= g.H) continue;
      const float* xrow = xc + (static_cast<size_t>(n) * g.H + hi) * g.W * g.C;
      const float* dyrow = dyk + (static_cast<size_t>(n) * g.Ho + ho) * g.Wo * g.K;
      for (int wo = wo0; wo < wo0 + bg.bwo; ++wo) {
        const int wi = wo * g.sw - g.pw + s * g.dw;
        if (wi < 0 || wi >= g.W) continue;
        acc = __fadd_rn(acc, __fmul_rn(xrow[static_cast<size_t>(wi) * g.C], dyrow[static_cast<size_t>(wo) * g.K]));
      }
    }
  }
  dw[e] = acc;
}

// dw on the matrix cores: dw[g Kg + k][j] = sum over pixels p of dy[p][g Kg + k] * col[p][j],
// j = (r, s, ci) the filter column, col the implicit im2col of x.  A workgroup of 8 waves
// computes 128 columns x 64 channels over its share of the pixels (chunks of 16), with the
// fprop kernel's staging, fragment layout and pipeline; the pixel range is split over
// workgroups.  With `part` a workgroup stores its partial tile at part[split] (a dw-shaped
// slice; with one split that slice is dw itself) and f32_sum_parts_kernel adds the splits in
// order; without it each adds its tile into dw (zeroed first) with float atomics.
struct GradArgs {
  const float* x;
  const float* dy;
  float* dw;
  float* part;  // split partial tiles (splits x K x By x Bx x kdim), or nullptr for float atomics
  Geom g;
  int P;       // pixels per filter block: N * bho * bwo
  int kdim;    // R * S * Cg
  int tn;      // channel tiles per group
  int tiles;   // column tiles * channel tiles per group
  int cps;     // 16-pixel chunks per split
  int By, Bx, bho, bwo;  // filter blocks (1 x 1 of Ho x Wo: a plain KRSC filter)
  FastDivM fd_tn, fd_tiles, fd_gt, fd_g;  // gt = G * By * Bx * tiles
  int gt;
};

// (n, ho, wo) of pixel index p within a block of rows x cols output positions, advanced one
// pixel or one chunk at a time
struct PixCursor {
  int n, ho, wo;
  __device__ __forceinline__ void init(int p, int rows, int cols) {
    const int rc = rows * cols;
    n = p / rc;
    const int r0 = p - n * rc;
    ho = r0 / cols;
    wo = r0 - ho * cols;
  }
  __device__ __forceinline__ void step(int rows, int cols) {
    if (++wo == cols) {
      wo = 0;
      if (++ho == rows) {
        ho = 0;
        ++n;
      }
    }
  }
  __device__ __forceinline__ void advance(int rows, int cols, int d) {
    wo += d;
    while (wo >= cols) {
      wo -= cols;
      if (++ho == rows) {
        ho = 0;
        ++n;
      }
    }
  }
};

__global__ void __launch_bounds__(64 * kF32Waves, 1) f32_grad_igemm_kernel(GradArgs a) {
  __shared__ v4f sA[2][kF32BM * 4];
  __shared__ v4f sB[2][kF32BN * 4];
  const Geom& g = a.g;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  const int lin = blockIdx.x;
  const int split = fdiv(lin, a.fd_gt);
  const int rem = lin - split * a.gt;
  const int gb = fdiv(rem, a.fd_tiles);  // block * G + group
  const int rem2 = rem - gb * a.tiles;
  const int blk = fdiv(gb, a.fd_g);
  const int grp = gb - blk * g.G;
  const int by0 = (blk / a.Bx) * a.bho;  // the block's first output row and column
  const int bx0 = (blk - (blk / a.Bx) * a.Bx) * a.bwo;
  const int nblk = a.By * a.Bx;
  const int tmi = fdiv(rem2, a.fd_tn);
  const int tni = rem2 - tmi * a.tn;
  const int m0 = tmi * kF32BM;
  const int n0 = tni * kF32BN;
  const int pb = split * a.cps * kF32KC;
  const int pe = min(a.P, pb + a.cps * kF32KC);
  if (pb >= pe) return;  // whole workgroup: an empty split (the host plans none)
  const int nch = (pe - pb + kF32KC - 1) / kF32KC;

  // A: filter column ja (r, s, ci), pixels pb + 16 c + 4 aq + e of chunk c
  const int ar = t >> 2;
  const int aq = t & 3;
  const int ja = min(m0 + ar, a.kdim - 1);
  const int tap = ja / g.Cg;
  const int aci = ja - tap * g.Cg;
  const int ar_ = tap / g.S;
  const int as_ = tap - ar_ * g.S;
  const float* xg = a.x + static_cast<size_t>(grp) * g.Cg + aci;
  PixCursor pc;
  pc.init(min(pb + 4 * aq, a.P - 1), a.bho, a.bwo);
  int cur_chunk = 0;
  // B: channel row, pixels pb + 16 c + 2 bp + e
  const int br = t >> 3;
  const int bp = t & 7;
  const int bk = grp * g.Kg + min(n0 + br, g.Kg - 1);
  const float* dyk = a.dy + bk;
  PixCursor bc;
  bc.init(min(pb + 2 * bp, a.P - 1), a.bho, a.bwo);
  auto dy_off = [&](const PixCursor& q) {
    return ((static_cast<size_t>(q.n) * g.Ho + by0 + q.ho) * g.Wo + bx0 + q.wo) * g.K;
  };
  const size_t ob0 = dy_off(bc);  // a valid offset for the pixels past the split

  auto load = [&](int c, v4f& va, v2f& vb, unsigned& oka, bool& okb) {
    if (cur_chunk < c) {  // chunks are loaded in order; a repeat of the last one does not advance
      pc.advance(a.bho, a.bwo, kF32KC);
      bc.advance(a.bho, a.bwo, kF32KC);
      ++cur_chunk;
    }
    PixCursor q = pc;
    oka = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (e > 0) q.step(a.bho, a.bwo);
      const int pp = pb + c * kF32KC + 4 * aq + e;
      const int hi = (by0 + q.ho) * g.sh - g.ph + ar_ * g.dh;
      const int wi = (bx0 + q.wo) * g.sw - g.pw + as_ * g.dw;
      const bool ok = pp < pe && hi >= 0 && hi < g.H && wi >= 0 && wi < g.W;
      oka |= static_cast<unsigned>(ok) << e;
      const size_t o = ok ? ((static_cast<size_t>(q.n) * g.H + hi) * g.W + wi) * g.C : 0;
      va[e] = xg[o];
    }
    const int pq = pb + c * kF32KC + 2 * bp;
    okb = pq < pe;  // pe - pb is not always even: the second pixel is checked at staging
    const bool ok2 = pq + 1 < pe;
    const size_t ob = okb ? dy_off(bc) : ob0;
    PixCursor q2 = bc;
    q2.step(a.bho, a.bwo);
    const size_t ob2 = ok2 ? dy_off(q2) : ob;
    vb = v2f{dyk[ob], dyk[ob2]};
  };
  const int sa_slot = f32_slot(ar, aq);
  const int sb_slot = f32_slot(br, bp >> 1);
  auto stage = [&](int buf, int c, const v4f& va, const v2f& vb, unsigned oka, bool live) {
    v4f v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (live && ((oka >> e) & 1u)) ? va[e] : 0.f;
    sA[buf][sa_slot] = v;
    const int pq = pb + c * kF32KC + 2 * bp;
    const v2f w2 = v2f{(live && pq < pe) ? vb[0] : 0.f, (live && pq + 1 < pe) ? vb[1] : 0.f};
    *(reinterpret_cast<v2f*>(&sB[buf][sb_slot]) + (bp & 1)) = w2;
  };

  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int fb0 = f32_slot(32 * wn + (lane & 15), lane >> 4);
  const int fb1 = f32_slot(32 * wn + 16 + (lane & 15), lane >> 4);
  const int fa0 = f32_slot(32 * wm + (lane & 15), lane >> 4);
  const int fa1 = f32_slot(32 * wm + 16 + (lane & 15), lane >> 4);
  v4f acc[2][2];
#pragma unroll
  for (int jn = 0; jn < 2; ++jn)
#pragma unroll
    for (int im = 0; im < 2; ++im) acc[jn][im] = v4f{0.f, 0.f, 0.f, 0.f};

  constexpr int P2 = kF32Depth;
  const int last = nch - 1;
  v4f va[P2];
  v2f vb[P2];
  unsigned oka[P2];
  bool okb[P2];
#pragma unroll
  for (int j = 0; j < P2; ++j) load(min(j, last), va[j], vb[j], oka[j], okb[j]);
  stage(0, 0, va[0], vb[0], oka[0], true);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  for (int c0 = 0; c0 < nch; c0 += P2) {
#pragma unroll
    for (int j = 0; j < P2; ++j) {
      const int c = c0 + j;
      load(min(c + P2, last), va[j], vb[j], oka[j], okb[j]);
      const int buf = c & 1;
      const v4f Bf[2] = {sB[buf][fb0], sB[buf][fb1]};
      const v4f Af[2] = {sA[buf][fa0], sA[buf][fa1]};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn)
#pragma unroll
          for (int im = 0; im < 2; ++im)
            acc[jn][im] = __builtin_amdgcn_mfma_f32_16x16x4f32(Bf[jn][kk], Af[im][kk], acc[jn][im], 0, 0, 0);
      const int j1 = (j + 1) % P2;
      stage(buf ^ 1, min(c + 1, last), va[j1], vb[j1], oka[j1], c + 1 <= last);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
  }

  // lane (c = lane % 16, q = lane / 16) of tile (jn, im): column m0 + 32 wm + 16 im + c,
  // channels n0 + 32 wn + 16 jn + 4 q .. + 3 of the group
#pragma unroll
  for (int jn = 0; jn < 2; ++jn) {
#pragma unroll
    for (int im = 0; im < 2; ++im) {
      const int jcol = m0 + 32 * wm + 16 * im + (lane & 15);
      const int ch = n0 + 32 * wn + 16 * jn + 4 * (lane >> 4);
      if (jcol >= a.kdim) continue;
      // dw[k][by][bx][j]
      if (a.part != nullptr) {
        float* pt = a.part + static_cast<size_t>(split) * g.K * nblk * a.kdim;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (ch + i < g.Kg)
            pt[(static_cast<size_t>(grp * g.Kg + ch + i) * nblk + blk) * a.kdim + jcol] = acc[jn][im][i];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (ch + i < g.Kg)
            unsafeAtomicAdd(a.dw + (static_cast<size_t>(grp * g.Kg + ch + i) * nblk + blk) * a.kdim + jcol,
                            acc[jn][im][i]);
      }
    }
  }
}

// Bias gradient of the blocked convolution, the sum of dy over every output position of a block
// (launch_block_grad_nhwc, cuda_kernels.cu:1112-1119, adds them all with float atomics), in a
// fixed order: f32_dbias_part_kernel sums runs of kDbiasChunk consecutive positions of a block
// ((n, lho, lwo) order) into part[blk][chunk][k], one thread per entry; f32_dbias_sum_kernel
// adds a slot's runs in chunk order (bias_mode 0: dbias[k][by][bx]) or every block's runs in
// block order (bias_mode 1: dbias[k][0][0], the other slots zero), starting from 0.
constexpr int kDbiasChunk = 256;

__global__ void __launch_bounds__(kDirectThreads) f32_dbias_part_kernel(const float* __restrict__ dy,
                                                                        float* __restrict__ part, Geom g,
                                                                        BlockGeom bg, int chunks, long long total) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  const int k = static_cast<int>(e % g.K);
  const long long t1 = e / g.K;
  const int ch = static_cast<int>(t1 % chunks);
  const int blk = static_cast<int>(t1 / chunks);
  const int ho0 = (blk / bg.Bx) * bg.bho;
  const int wo0 = (blk - (blk / bg.Bx) * bg.Bx) * bg.bwo;
  const int P = g.N * bg.bho * bg.bwo;
  const int p0 = ch * kDbiasChunk;
  const int p1 = min(P, p0 + kDbiasChunk);
  const int rc = bg.bho * bg.bwo;
  int n = p0 / rc;
  int lho = (p0 - n * rc) / bg.bwo;
  int lwo = p0 - n * rc - lho * bg.bwo;
  float acc = 0.0f;
  for (int p = p0; p < p1; ++p) {
    acc = __fadd_rn(acc, dy[((static_cast<size_t>(n) * g.Ho + ho0 + lho) * g.Wo + wo0 + lwo) * g.K + k]);
    if (++lwo == bg.bwo) {
      lwo = 0;
      if (++lho == bg.bho) {
        lho = 0;
        ++n;
      }
    }
  }
  part[e] = acc;
}

__global__ void __launch_bounds__(kDirectThreads) f32_dbias_sum_kernel(const float* __restrict__ part,
                                                                       float* __restrict__ dbias, int K, int nblk,
                                                                       int chunks, int bias_mode, long long total) {
  const long long e = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x;
  if (e >= total) return;
  const int k = static_cast<int>(e / nblk);
  const int blk = static_cast<int>(e - static_cast<long long>(k) * nblk);
  float acc = 0.0f;
  if (bias_mode == 0 || blk == 0) {
    const int b0 = bias_mode == 0 ? blk : 0;
    const int b1 = bias_mode == 0 ? blk + 1 : nblk;
    for (int b = b0; b < b1; ++b)
      for (int c = 0; c < chunks; ++c) acc = __fadd_rn(acc, part[(static_cast<size_t>(b) * chunks + c) * K + k]);
  }
  dbias[e] = acc;
}

__global__ void __launch_bounds__(kDirectThreads) f32_zero_kernel(float* __restrict__ p, long long count) {
  const long long stride = static_cast<long long>(gridDim.x) * kDirectThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kDirectThreads + threadIdx.x; i < count; i += stride)
    p[i] = 0.0f;
}

}  // namespace

bool f32_grad_igemm_eligible(const Geom& g, const BlockGeom& bg, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  const long long px = static_cast<long long>(g.N) * bg.bho * bg.bwo;
  const long long in = static_cast<long long>(g.N) * g.H * g.W * g.C;
  const long long kdim = static_cast<long long>(g.R) * g.S * g.Cg;
  if (px == 0 || in == 0 || kdim == 0 || g.Kg == 0) return no("fp32 grad on MFMA needs non-empty x, dy and dw");
  if (px >= (1LL << 31) - 64 || kdim >= (1LL << 31) - kF32BM) return no("fp32 grad on MFMA extents exceed int32");
  const long long tiles = ((kdim + kF32BM - 1) / kF32BM) * ((g.Kg + kF32BN - 1) / kF32BN) * g.G *
                          static_cast<long long>(bg.By) * bg.Bx;
  if (tiles > (1LL << 20)) return no("fp32 grad on MFMA: more than 2^20 output tiles");
  return true;
}

namespace {

// Pixel split of the MFMA grad: about `target` workgroups, at least 8 chunks (128 pixels) each,
// every split non-empty.  The float-atomic form aims at 2048 workgroups; the ordered form at
// 1024, which halves its partial tiles (workspace and the summing pass).
struct GradSplit {
  int cps;           // 16-pixel chunks per split
  long long splits;  // non-empty splits
};
GradSplit grad_split(const Geom& g, const BlockGeom& bg, bool ordered) {
  const long long P = static_cast<long long>(g.N) * bg.bho * bg.bwo;
  const long long kdim = static_cast<long long>(g.R) * g.S * g.Cg;
  const long long gt = ((kdim + kF32BM - 1) / kF32BM) * ((g.Kg + kF32BN - 1) / kF32BN) * g.G *
                       static_cast<long long>(bg.By) * bg.Bx;
  const long long target = ordered ? 1024 : 2048;
  const long long chunks = (P + kF32KC - 1) / kF32KC;
  long long splits = std::max(1LL, std::min((target + gt - 1) / gt, (chunks + 7) / 8));
  GradSplit s;
  s.cps = static_cast<int>((chunks + splits - 1) / splits);
  s.splits = (chunks + s.cps - 1) / s.cps;  // every split holds at least one chunk
  return s;
}

void launch_sum_parts(const float* part, float* dw, long long count, long long nparts, hipStream_t stream) {
  const unsigned blocks = static_cast<unsigned>(std::min<long long>((count + kDirectThreads - 1) / kDirectThreads, 8192));
  hipLaunchKernelGGL(f32_sum_parts_kernel, dim3(blocks), dim3(kDirectThreads), 0, stream, part, dw, count,
                     static_cast<int>(nparts));
}

}  // namespace

size_t f32_grad_igemm_workspace(const Geom& g, const BlockGeom& bg) {
  const GradSplit sp = grad_split(g, bg, true);
  if (sp.splits <= 1) return 0;
  return static_cast<size_t>(sp.splits) * g.K * bg.By * bg.Bx * g.R * g.S * g.Cg * sizeof(float);
}

hipError_t launch_f32_grad_igemm(const Geom& g, const BlockGeom& bg, const float* x, const float* dy, float* dw,
                                 float* ws, bool ordered, hipStream_t stream) {
  GradArgs a;
  a.x = x; a.dy = dy; a.dw = dw; a.g = g;
  a.By = bg.By; a.Bx = bg.Bx; a.bho = bg.bho; a.bwo = bg.bwo;
  a.P = g.N * bg.bho * bg.bwo;
  a.kdim = g.R * g.S * g.Cg;
  a.tn = (g.Kg + kF32BN - 1) / kF32BN;
  a.tiles = ((a.kdim + kF32BM - 1) / kF32BM) * a.tn;
  a.gt = a.tiles * g.G * bg.By * bg.Bx;
  const GradSplit sp = grad_split(g, bg, ordered);
  a.cps = sp.cps;
  a.fd_tn = fastdiv_m(a.tn);
  a.fd_tiles = fastdiv_m(a.tiles);
  a.fd_gt = fastdiv_m(a.gt);
  a.fd_g = fastdiv_m(g.G);
  const long long count = static_cast<long long>(g.K) * bg.By * bg.Bx * a.kdim;
  const unsigned blocks = static_cast<unsigned>(sp.splits * a.gt);
  if (ordered) {
    // one split writes dw directly; more write their partial tiles, summed in split order
    a.part = sp.splits == 1 ? dw : ws;
    hipLaunchKernelGGL(f32_grad_igemm_kernel, dim3(blocks), dim3(64 * kF32Waves), 0, stream, a);
    if (sp.splits > 1) launch_sum_parts(ws, dw, count, sp.splits, stream);
    return hipGetLastError();
  }
  a.part = nullptr;
  const unsigned zb = static_cast<unsigned>(std::min<long long>((count + kDirectThreads - 1) / kDirectThreads, 4096));
  hipLaunchKernelGGL(f32_zero_kernel, dim3(zb), dim3(kDirectThreads), 0, stream, dw, count);
  hipLaunchKernelGGL(f32_grad_igemm_kernel, dim3(blocks), dim3(64 * kF32Waves), 0, stream, a);
  return hipGetLastError();
}

bool f32_depthwise_eligible(const Geom& g, const void* x, const void* y) {
  return g.Cg == 1 && g.Kg == 1 && g.C % 4 == 0 && static_cast<long long>(g.R) * g.S * g.C <= kDwLdsFloats &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
}

hipError_t launch_f32_depthwise(const Geom& g, const float* x, const float* w, float* y, hipStream_t stream) {
  const long long total = static_cast<long long>(g.N) * g.Ho * g.Wo * (g.C / 4);
  if (total == 0) return hipSuccess;
  const long long blocks = (total + kDirectThreads - 1) / kDirectThreads;
  hipLaunchKernelGGL(f32_depthwise_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream, x, w,
                     y, g, total, make_split3(g.C / 4, g.Wo, g.Ho));
  return hipGetLastError();
}

bool f32_bprop_direct4_eligible(const Geom& g, const void* w, const void* dx) {
  return g.Cg % 4 == 0 && g.Cg > 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(dx) & 15u) == 0;
}

bool f32_depthwise_bprop_eligible(const Geom& g, const void* dy, const void* dx) {
  return g.Cg == 1 && g.Kg == 1 && g.C % 4 == 0 && g.C > 0 && static_cast<long long>(g.R) * g.S * g.C <= kDwLdsFloats &&
         (reinterpret_cast<uintptr_t>(dy) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dx) & 15u) == 0;
}

hipError_t launch_f32_depthwise_bprop(const Geom& g, const float* dy, const float* w, float* dx, hipStream_t stream) {
  const long long total = static_cast<long long>(g.N) * g.H * g.W * (g.C / 4);
  if (total == 0) return hipSuccess;
  const long long blocks = (total + kDirectThreads - 1) / kDirectThreads;
  hipLaunchKernelGGL(f32_depthwise_bprop_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream,
                     dy, w, dx, g, total, make_split3(g.C / 4, g.W, g.H));
  return hipGetLastError();
}

hipError_t launch_f32_bprop_direct(const Geom& g, const BlockGeom& bg, const float* dy, const float* w, float* dx,
                                   hipStream_t stream) {
  if (f32_bprop_direct4_eligible(g, w, dx)) {
    const long long quads = static_cast<long long>(g.N) * g.H * g.W * (g.C / 4);
    if (quads == 0) return hipSuccess;
    const long long qblocks = (quads + kDirectThreads - 1) / kDirectThreads;
    hipLaunchKernelGGL(f32_bprop_direct4_kernel, dim3(static_cast<unsigned>(qblocks)), dim3(kDirectThreads), 0, stream,
                       dy, w, dx, g, bg, quads, make_split3(g.C / 4, g.W, g.H));
    return hipGetLastError();
  }
  const long long total = static_cast<long long>(g.N) * g.H * g.W * g.C;
  if (total == 0) return hipSuccess;
  const long long blocks = (total + kDirectThreads - 1) / kDirectThreads;
  hipLaunchKernelGGL(f32_bprop_direct_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream,
                     dy, w, dx, g, bg, total, make_split3(g.C, g.W, g.H));
  return hipGetLastError();
}

hipError_t launch_f32_grad_direct(const Geom& g, const BlockGeom& bg, const float* x, const float* dy, float* dw,
                                  hipStream_t stream) {
  const long long total = static_cast<long long>(g.K) * bg.By * bg.Bx * g.R * g.S * g.Cg;
  if (total == 0) return hipSuccess;
  const long long blocks = (total + kDirectThreads - 1) / kDirectThreads;
  hipLaunchKernelGGL(f32_grad_direct_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream, x,
                     dy, dw, g, bg, total);
  return hipGetLastError();
}

size_t f32_block_dbias_workspace(const Geom& g, const BlockGeom& bg) {
  const long long P = static_cast<long long>(g.N) * bg.bho * bg.bwo;
  const long long chunks = (P + kDbiasChunk - 1) / kDbiasChunk;
  return static_cast<size_t>(bg.By) * bg.Bx * chunks * g.K * sizeof(float);
}

hipError_t launch_f32_block_dbias(const Geom& g, const BlockGeom& bg, const float* dy, float* dbias, int bias_mode,
                                  float* ws, hipStream_t stream) {
  const int P = g.N * bg.bho * bg.bwo;
  const int chunks = (P + kDbiasChunk - 1) / kDbiasChunk;
  const long long parts = static_cast<long long>(bg.By) * bg.Bx * chunks * g.K;
  if (parts > 0) {
    const long long blocks = (parts + kDirectThreads - 1) / kDirectThreads;
    hipLaunchKernelGGL(f32_dbias_part_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream,
                       dy, ws, g, bg, chunks, parts);
  }
  const long long slots = static_cast<long long>(g.K) * bg.By * bg.Bx;
  if (slots > 0) {
    const long long blocks = (slots + kDirectThreads - 1) / kDirectThreads;
    hipLaunchKernelGGL(f32_dbias_sum_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream, ws,
                       dbias, g.K, bg.By * bg.Bx, chunks, bias_mode, slots);
  }
  return hipGetLastError();
}

namespace {

// Output regions of the implicit GEMM (F32Args): forward, the filter blocks themselves; the
// transposed form, By x Bx regions of ceil(Ho / By) x ceil(Wo / Bx) positions (the last ones
// clipped), so that most tiles reach the input positions of one filter block only.
struct Regions {
  int ry, rx, rh, rw;
};
Regions fprop_regions(const BlockGeom& bg) { return Regions{bg.By, bg.Bx, bg.bho, bg.bwo}; }
Regions bprop_regions(const Geom& b, const BlockGeom& bg) {
  return Regions{bg.By, bg.Bx, (b.Ho + bg.By - 1) / bg.By, (b.Wo + bg.Bx - 1) / bg.Bx};
}

bool igemm_fits(const Geom& g, const Regions& rg, const void* x, const void* w, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (g.Cg % 4 != 0) return no("fp32 implicit GEMM needs (c/groups) % 4 == 0");
  if (g.H == 0 || g.W == 0) return no("fp32 implicit GEMM needs a non-empty input image");
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(w) & 15u) != 0) {
    return no("fp32 implicit GEMM needs 16-byte aligned x and w");
  }
  const long long m = static_cast<long long>(g.N) * rg.rh * rg.rw;
  const long long kdim = static_cast<long long>(g.R) * g.S * g.Cg;
  if (m >= (1LL << 31) - 2 * kF32BM || kdim >= (1LL << 31) - kF32KC) {
    return no("fp32 implicit GEMM extents exceed int32");
  }
  const long long tiles =
      ((m + kF32BM - 1) / kF32BM) * ((g.Kg + kF32BN - 1) / kF32BN) * g.G * static_cast<long long>(rg.ry) * rg.rx;
  if (tiles > (1LL << 22)) return no("fp32 implicit GEMM grid exceeds 2^22 workgroups");
  return true;
}

hipError_t f32_igemm_launch(const Geom& g, const BlockGeom& bg, const Regions& rg, const float* x, const float* w,
                            const float* bias, int bias_mode, float* y, bool transposed, hipStream_t stream) {
  F32Args a;
  a.x = x; a.w = w; a.y = y; a.bias = bias; a.g = g;
  a.ow_taps = g.R * g.S;
  a.ow_cg = g.Kg;
  a.ry = rg.ry; a.rx = rg.rx; a.rh = rg.rh; a.rw = rg.rw;
  a.By = bg.By; a.Bx = bg.Bx; a.bho = bg.bho; a.bwo = bg.bwo;
  a.bias_mode = bias_mode;
  a.nfast = transposed && bg.By * bg.Bx > 1 ? 1 : 0;
  a.M = g.N * rg.rh * rg.rw;
  a.kdim = g.R * g.S * g.Cg;
  a.nchunks = (a.kdim + kF32KC - 1) / kF32KC;
  const bool narrow = g.Kg <= 32;  // 256 pixels x 32 channels per workgroup
  const int bm = narrow ? 256 : kF32BM, bn = narrow ? 32 : kF32BN;
  a.tn = (g.Kg + bn - 1) / bn;
  a.tiles = ((a.M + bm - 1) / bm) * a.tn;
  a.fd_tn = fastdiv_m(a.tn);
  a.fd_tiles = fastdiv_m(a.tiles);
  a.fd_regions = fastdiv_m(rg.ry * rg.rx);
  a.fd_rx = fastdiv_m(rg.rx);
  const unsigned blocks = static_cast<unsigned>(a.tiles) * static_cast<unsigned>(g.G) *
                          static_cast<unsigned>(rg.ry * rg.rx);
  const dim3 grid(blocks), block(64 * kF32Waves);
  if (transposed && a.By * a.Bx > 1) {
    if (narrow) hipLaunchKernelGGL((f32_igemm_kernel<kTransBlocked, 32>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((f32_igemm_kernel<kTransBlocked, 64>), grid, block, 0, stream, a);
  } else if (transposed) {
    if (narrow) hipLaunchKernelGGL((f32_igemm_kernel<kTrans, 32>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((f32_igemm_kernel<kTrans, 64>), grid, block, 0, stream, a);
  } else {
    if (narrow) hipLaunchKernelGGL((f32_igemm_kernel<kFwd, 32>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((f32_igemm_kernel<kFwd, 64>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}
}  // namespace

bool f32_igemm_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, std::string* why) {
  return igemm_fits(g, fprop_regions(bg), x, w, why);
}

hipError_t launch_f32_igemm(const Geom& g, const BlockGeom& bg, const float* x, const float* w, const float* bias,
                            int bias_mode, float* y, hipStream_t stream) {
  return f32_igemm_launch(g, bg, fprop_regions(bg), x, w, bias, bias_mode, y, false, stream);
}

// The bprop of a stride-1 convolution g as the forward convolution of dy (N x Ho x Wo x K)
// with the flipped, channel-transposed filter: padding dilation * (R - 1) - pad, stride 1,
// the same dilation and groups, output N x H x W x C.
Geom f32_bprop_as_fprop(const Geom& g) {
  Geom b = g;
  b.H = g.Ho; b.W = g.Wo; b.C = g.K;
  b.Ho = g.H; b.Wo = g.W; b.K = g.C;
  b.ph = g.dh * (g.R - 1) - g.ph;
  b.pw = g.dw * (g.S - 1) - g.pw;
  b.Cg = g.Kg; b.Kg = g.Cg;
  return b;
}

bool f32_bprop_igemm_eligible(const Geom& g, const BlockGeom& bg, const void* dy, const void* w, std::string* why) {
  if (g.sh != 1 || g.sw != 1) {
    if (why) *why = "fp32 bprop on MFMA needs stride 1";
    return false;
  }
  const Geom b = f32_bprop_as_fprop(g);
  return igemm_fits(b, bprop_regions(b, bg), dy, w, why);
}

// Rows of the transposed filter are the original's input channels (b.Kg = g.Cg), its reduction
// (r', s', ko < g.Kg = b.Cg); f32_igemm_launch takes ow_taps = R * S and ow_cg = b.Kg from b.
// The filter blocks partition dy (bg: blocks of the original output).
hipError_t launch_f32_bprop_igemm(const Geom& g, const BlockGeom& bg, const float* dy, const float* w, float* dx,
                                  hipStream_t stream) {
  const Geom b = f32_bprop_as_fprop(g);
  return f32_igemm_launch(b, bg, bprop_regions(b, bg), dy, w, nullptr, 0, dx, true, stream);
}

hipError_t launch_f32_direct(const Geom& g, const BlockGeom& bg, const float* x, const float* w, const float* bias,
                             int bias_mode, float* y, hipStream_t stream) {
  const long long total = static_cast<long long>(g.N) * g.Ho * g.Wo * g.K;
  if (total == 0) return hipSuccess;
  const long long blocks = (total + kDirectThreads - 1) / kDirectThreads;
  hipLaunchKernelGGL(f32_direct_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream, x, w,
                     y, g, bg, bias, bias_mode, total, make_split3(g.K, g.Wo, g.Ho));
  return hipGetLastError();
}

bool f32_depthwise_grad_eligible(const Geom& g, const void* x, const void* dy) {
  return g.Cg == 1 && g.Kg == 1 && g.C % 4 == 0 && g.R * g.S <= kDwGradTaps && g.R * g.S > 0 && g.H > 0 &&
         g.W > 0 && static_cast<long long>(g.N) * g.Ho * g.Wo < (1LL << 31) - kDwGradPix &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dy) & 15u) == 0;
}

size_t f32_depthwise_grad_workspace(const Geom& g) {
  const long long P = static_cast<long long>(g.N) * g.Ho * g.Wo;
  const long long runs = (P + kDwGradPix - 1) / kDwGradPix;
  if (runs <= 1) return 0;
  return static_cast<size_t>(runs) * g.K * g.R * g.S * sizeof(float);
}

hipError_t launch_f32_depthwise_grad(const Geom& g, const float* x, const float* dy, float* dw, float* ws,
                                     bool ordered, hipStream_t stream) {
  const int P = g.N * g.Ho * g.Wo;
  const long long count = static_cast<long long>(g.K) * g.R * g.S;
  const long long runs = (static_cast<long long>(P) + kDwGradPix - 1) / kDwGradPix;
  const long long total = runs * (g.C / 4);
  if (!ordered || runs == 0) {
    const unsigned zb = static_cast<unsigned>(std::min<long long>((count + kDirectThreads - 1) / kDirectThreads, 4096));
    hipLaunchKernelGGL(f32_zero_kernel, dim3(zb), dim3(kDirectThreads), 0, stream, dw, count);
  }
  if (total == 0) return hipGetLastError();
  const long long blocks = (total + kDirectThreads - 1) / kDirectThreads;
  // ordered: one run writes dw directly; more write their partial sums, added in run order
  float* part = !ordered ? nullptr : (runs == 1 ? dw : ws);
  hipLaunchKernelGGL(f32_depthwise_grad_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kDirectThreads), 0, stream,
                     x, dy, dw, part, g, P, total);
  if (ordered && runs > 1) launch_sum_parts(ws, dw, count, runs, stream);
  return hipGetLastError();
}

}  // namespace miq
