// int8 MFMA convolution for thin-channel layers (network stems, C < 16).
//
// With C < 16 a tap holds too few bytes for the chunk-per-tap reduction of the implicit
// GEMM kernel.  Instead the reduction runs over filter ROWS: for output pixel (ho, wo)
// and filter row r, the S taps x C channels are S*C contiguous bytes of the NHWC input
// row (unit dilation along W) and S*C contiguous bytes of the KRSC filter.  Each filter
// row is padded to a slot of RowB = 16 or 32 bytes (one or two 16-byte chunks); the
// padding bytes of the filter are zero, so the input bytes read past the window do not
// contribute.  For a 7x7x3 stem that is 7 slots of 32 bytes = 4 MFMA K-blocks of 64
// (57% of the MFMA work is useful), against an HBM floor that the 64-channel int8
// output dominates.
//
// A workgroup owns RB whole output rows of one image and 64 output channels.  It stages
// the filter slice (contiguous in KRSC) and the HR input rows (full width, with zero
// columns for the padding) into LDS; every lane then assembles its 16-byte operands from
// arbitrary byte offsets with aligned dword reads and v_alignbyte_b32.  The filter
// fragments stay in registers for the whole tile.

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kThreads = 256;
constexpr int kNseg = 4;
constexpr int kStageBatch = 8;  // dword loads in flight per thread while staging
constexpr int kLdsBudget = 64 * 1024;

struct StemArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  void* y;
  int H, W, C, K, R, S, Ho, Wo;
  int ph, pw, sh, sw, dh;
  int SC, RSC;      // bytes of one filter row, of one output channel's filter
  int CPR, NQ;      // 16-byte chunks per row slot, R * CPR
  int RB, tiles_h;  // output rows per tile
  int PL, P;        // left zero pad and pitch (bytes) of one staged input row
  int w_off;        // LDS byte offset of the staged filter slice
  int w_bytes;      // LDS bytes reserved for it
  int ep_off;       // LDS byte offset of the 64 biases and 64 multipliers
  int row_dw;       // input rows are dword aligned (W*C % 4 == 0)
  float act_scale;
  int relu;
};

template <int KB, int EPI>
__global__ void __launch_bounds__(kThreads)
i8_stem_kernel(StemArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = blockIdx.x / a.tiles_h;
  const int th = blockIdx.x - n * a.tiles_h;
  const int k0 = blockIdx.y * 64;
  const int ho0 = th * a.RB;
  const int rows = min(a.RB, a.Ho - ho0);
  const int HR = (rows - 1) * a.sh + (a.R - 1) * a.dh + 1;
  const int hi0 = ho0 * a.sh - a.ph;

  // ---- filter slice [k0, k0+kn) (contiguous bytes of the KRSC filter) and the input rows
  // hi0 .. hi0+HR-1 (full width, zero columns left and right) -> LDS; every load of both is
  // issued before the first LDS write waits on it ----
  unsigned char* wl = smem + a.w_off;
  {
    const int kn = min(64, a.K - k0);
    const int L = kn * a.RSC;  // 4-aligned start: k0 * RSC is a multiple of 64
    const unsigned char* wsrc = reinterpret_cast<const unsigned char*>(a.w) + static_cast<size_t>(k0) * a.RSC;
    const int ndw_w = a.w_bytes >> 2;
    const int dw_per_row = a.P >> 2;
    const int ndw_x = HR * dw_per_row;
    const int rowb = a.W * a.C;
    const unsigned char* ximg = reinterpret_cast<const unsigned char*>(a.x) + static_cast<size_t>(n) * a.H * rowb;
    const int total = ndw_x + ndw_w;
    for (int base = tid; base < total; base += kThreads * kStageBatch) {
      unsigned tmp[kStageBatch];
#pragma unroll
      for (int u = 0; u < kStageBatch; ++u) {
        const int i = base + u * kThreads;
        unsigned v = 0;
        if (i < ndw_x) {
          const int hr = i / dw_per_row;
          const int b = (i - hr * dw_per_row) * 4 - a.PL;  // byte index in the input row
          const int hi = hi0 + hr;
          if (static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) && b + 4 > 0 && b < rowb) {
            const unsigned char* src = ximg + static_cast<size_t>(hi) * rowb;
            if (a.row_dw && b >= 0 && b + 4 <= rowb) {
              v = *reinterpret_cast<const unsigned*>(src + b);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (b + e >= 0 && b + e < rowb) v |= static_cast<unsigned>(src[b + e]) << (8 * e);
            }
          }
        } else if (i < total) {
          const int b = (i - ndw_x) * 4;
          if (b + 4 <= L) {
            v = *reinterpret_cast<const unsigned*>(wsrc + b);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (b + e < L) v |= static_cast<unsigned>(wsrc[b + e]) << (8 * e);
          }
        }
        tmp[u] = v;
      }
#pragma unroll
      for (int u = 0; u < kStageBatch; ++u) {
        const int i = base + u * kThreads;
        if (i < ndw_x) {
          reinterpret_cast<unsigned*>(smem)[i] = tmp[u];
        } else if (i < total) {
          reinterpret_cast<unsigned*>(wl)[i - ndw_x] = tmp[u];
        }
      }
    }
  }
  int32_t* ep_bias = reinterpret_cast<int32_t*>(smem + a.ep_off);
  float* ep_mult = reinterpret_cast<float*>(smem + a.ep_off) + 64;
  stage_requant<EPI>(Requant{a.bias, a.wscale, a.act_scale, a.relu}, k0, a.K - k0, 64, ep_bias, ep_mult);
  __syncthreads();

  const int row_l = lane & 15;
  const int grp_l = lane >> 4;

  // ---- filter fragments, resident in registers for the whole tile ----
  v4i A[KB][4];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    const int q = 4 * b + grp_l;
    const int r = q / a.CPR;
    const int h = q - r * a.CPR;
    // bytes h*16 + e of the row slot exist only below SC
    const int nvalid = min(16, max(0, a.SC - h * 16));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kl = 16 * (row_l >> 2) + 4 * j + (row_l & 3);
      v4i v = {0, 0, 0, 0};
      if (q < a.NQ && k0 + kl < a.K && nvalid > 0) {
        v = lds_load16_unaligned(wl, kl * a.RSC + r * a.SC + h * 16);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int keep = min(4, max(0, nvalid - 4 * d));  // bytes of dword d to keep
          const unsigned m = keep >= 4 ? 0xffffffffu : ((1u << (8 * keep)) - 1u);
          v[d] = static_cast<int>(static_cast<unsigned>(v[d]) & m);
        }
      }
      A[b][j] = v;
    }
  }

  const int npix = rows * a.Wo;
  const int nseg = (npix + 15) >> 4;
  const int kc0 = 16 * grp_l;  // first of this lane's 16 output channels (relative to k0)
  const bool kvalid = k0 + kc0 < a.K;
  const bool full = (k0 + kc0 + 16 <= a.K) && ((a.K & 15) == 0);

  for (int sg0 = wave * kNseg; sg0 < nseg; sg0 += 4 * kNseg) {
    int ob[kNseg];
    bool pv[kNseg];
#pragma unroll
    for (int i = 0; i < kNseg; ++i) {
      const int p = (sg0 + i) * 16 + row_l;
      pv[i] = p < npix;
      const int lho = p / a.Wo;
      const int lwo = p - lho * a.Wo;
      ob[i] = pv[i] ? (lho * a.sh) * a.P + a.PL + (lwo * a.sw - a.pw) * a.C : 0;
    }
    v4i acc[4][kNseg];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < kNseg; ++i) acc[j][i] = v4i{0, 0, 0, 0};

#pragma unroll
    for (int b = 0; b < KB; ++b) {
      const int q = 4 * b + grp_l;
      const int r = q / a.CPR;
      const int h = q - r * a.CPR;
      const bool qv = q < a.NQ;
      const int off = r * a.dh * a.P + h * 16;
      v4i B[kNseg];
#pragma unroll
      for (int i = 0; i < kNseg; ++i) {
        v4i v = {0, 0, 0, 0};
        if (qv && pv[i]) v = lds_load16_unaligned(smem, ob[i] + off);
        B[i] = v;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < kNseg; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[i], acc[j][i], 0, 0, 0);
    }

    if (!kvalid) continue;
#pragma unroll
    for (int i = 0; i < kNseg; ++i) {
      if (!pv[i]) continue;
      const int p = (sg0 + i) * 16 + row_l;
      const int lho = p / a.Wo;
      const int lwo = p - lho * a.Wo;
      const size_t opix = (static_cast<size_t>(n) * a.Ho + (ho0 + lho)) * a.Wo + lwo;
      const v4i frag[4] = {acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
      store16<EPI>(a.y, opix * a.K + k0 + kc0, frag, k0 + kc0, a.K, full, ep_bias + kc0, ep_mult + kc0, a.relu);
    }
  }
}

struct StemPlan {
  int RowB, CPR, NQ, KB;
  int RB, tiles_h;
  int PL, P, w_off, w_bytes, ep_off;
  size_t lds;
};

int round_up(int v, int m) { return (v + m - 1) / m * m; }

bool make_plan(const Geom& g, StemPlan* pl) {
  const int SC = g.S * g.C;
  pl->RowB = SC <= 16 ? 16 : 32;
  pl->CPR = pl->RowB / 16;
  pl->NQ = g.R * pl->CPR;
  pl->KB = (pl->NQ + 3) / 4;
  if (pl->KB > 4) return false;
  pl->PL = round_up(std::max(0, g.pw) * g.C, 16);
  // Largest byte any lane reads in a staged row: window start of the last output column
  // plus the row slot plus the 4-byte over-read of the unaligned LDS loader.
  const long long last = static_cast<long long>(pl->PL) + (static_cast<long long>(g.Wo - 1) * g.sw - g.pw) * g.C +
                         pl->RowB + 4;
  const long long need = std::max<long long>(static_cast<long long>(pl->PL) + static_cast<long long>(g.W) * g.C, last);
  if (need > kLdsBudget) return false;
  pl->P = round_up(static_cast<int>(need), 16);
  const int RSC = g.R * SC;
  pl->w_bytes = round_up(64 * RSC + 32, 16);
  // target about 16 segments (256 pixels) per tile
  int RB = std::max(1, std::min(g.Ho, 256 / std::max(1, g.Wo)));
  auto lds_for = [&](int rb) {
    const long long HR = static_cast<long long>(rb - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
    return HR * pl->P + pl->w_bytes + 512;
  };
  while (RB > 1 && lds_for(RB) > kLdsBudget) --RB;
  if (lds_for(RB) > kLdsBudget) return false;
  pl->RB = RB;
  pl->tiles_h = (g.Ho + RB - 1) / RB;
  const long long HR = static_cast<long long>(RB - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
  pl->w_off = static_cast<int>(HR * pl->P);
  pl->ep_off = pl->w_off + pl->w_bytes;
  pl->lds = static_cast<size_t>(lds_for(RB));
  return true;
}

template <int EPI>
void launch_kb(const StemArgs& a, const StemPlan& pl, int N, int K, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(N * pl.tiles_h), static_cast<unsigned>((K + 63) / 64));
  switch (pl.KB) {
    case 1: hipLaunchKernelGGL((i8_stem_kernel<1, EPI>), grid, dim3(kThreads), pl.lds, stream, a); break;
    case 2: hipLaunchKernelGGL((i8_stem_kernel<2, EPI>), grid, dim3(kThreads), pl.lds, stream, a); break;
    case 3: hipLaunchKernelGGL((i8_stem_kernel<3, EPI>), grid, dim3(kThreads), pl.lds, stream, a); break;
    default: hipLaunchKernelGGL((i8_stem_kernel<4, EPI>), grid, dim3(kThreads), pl.lds, stream, a); break;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool stem_eligible(const Geom& g, const void* x, const void* w, const void* y, Epi epi, std::string* why) {
  (void)epi;
  auto no = [&](const char* m) { if (why) *why = m; return false; };
  if (g.G != 1) return no("stem kernel needs groups == 1");
  if (g.C < 1 || g.C >= 16) return no("stem kernel is for 1 <= c < 16");
  if (g.S * g.C > 32) return no("stem kernel needs s*c <= 32");
  if (g.dw != 1) return no("stem kernel needs dilation_w == 1");
  if (g.sh < 1 || g.sw < 1 || g.dh < 1) return no("stem kernel needs stride and dilation_h >= 1");
  if (g.ph < 0 || g.pw < 0) return no("stem kernel needs non-negative padding");
  if (g.R < 1 || g.S < 1 || g.K < 1) return no("stem kernel needs a non-empty filter");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y)) return no("stem kernel needs 16-byte aligned tensors");
  StemPlan pl;
  if (!make_plan(g, &pl)) return no("stem kernel tile does not fit in LDS or r*slots exceeds 4 K-blocks");
  if (static_cast<long long>(g.N) * pl.tiles_h > 0x7fffffffLL || (g.K + 63) / 64 > 65535) return no("grid too large");
  return true;
}

hipError_t launch_i8_stem(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  StemPlan pl;
  if (!make_plan(g, &pl)) return hipErrorInvalidConfiguration;
  StemArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.R = g.R; a.S = g.S; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.sh = g.sh; a.sw = g.sw; a.dh = g.dh;
  a.SC = g.S * g.C; a.RSC = g.R * a.SC;
  a.CPR = pl.CPR; a.NQ = pl.NQ;
  a.RB = pl.RB; a.tiles_h = pl.tiles_h;
  a.PL = pl.PL; a.P = pl.P; a.w_off = pl.w_off; a.w_bytes = pl.w_bytes; a.ep_off = pl.ep_off;
  a.row_dw = ((g.W * g.C) % 4 == 0) ? 1 : 0;
  a.act_scale = rq.act_scale;
  a.relu = rq.relu;
  switch (epi) {
    case kEpiI8: launch_kb<kEpiI8>(a, pl, g.N, g.K, stream); break;
    case kEpiAcc32: launch_kb<kEpiAcc32>(a, pl, g.N, g.K, stream); break;
    default: launch_kb<kEpiF32>(a, pl, g.N, g.K, stream); break;
  }
  return hipGetLastError();
}

}  // namespace miq
