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
//
// Row-band variant (i8_stem_band_kernel, used when the shape allows it).  A workgroup of
// 8 waves owns a band of BH output rows of one image and 64 channels, about one band per
// CU.  Its loads are buffer_load_dwordx4 ... lds (global -> LDS, no registers): the
// filter slice as contiguous kilobytes, and every input row as P/1024 kilobyte
// instructions whose lane l carries row bytes [1024m + 16l - PLB, +16).  A lane whose
// bytes lie left or right of the row, or a row outside the image, gets an offset past
// num_records and writes zeros, so the padding costs nothing.  Then each wave takes
// 16-pixel segments of the band in turn: its K-blocks' operands come from the staged rows
// at arbitrary byte offsets (read one segment ahead), and the int8 result of 16 channels
// per lane leaves in one 16-byte buffer store.

#include "qconv_device.h"

#include <algorithm>
#include <atomic>

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

int round_up(int v, int m) { return (v + m - 1) / m * m; }

// ---------------------------------------------------------------------------------------
// Row-band variant

constexpr int kSbWaves = 8;
constexpr int kSbLds = 160 * 1024;

struct StemBandArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  void* y;
  int H, W, C, K, Ho, Wo;
  int ph, pw, sh, sw, dh;
  int SC, RSC, CPR, NQ;  // filter row bytes, filter bytes per channel, chunks per row slot, R * CPR
  int BH, bands_per_img, nbands, nblocks;
  int SEGR;              // 16-pixel segments per output row
  int P, PLB, rows_ld;   // staged row pitch (bytes, multiple of 1024), its left pad, loads per row
  int HR;                // staged input rows per band
  int nfilt;             // filter load instructions
  int filt_lds, ep_lds, halo_lds;  // LDS byte offsets
  int slot_lds;          // LDS byte offset of the filter's 16-byte operand slots (16 KB)
  float act_scale;
  int relu;
  FastDivM fd_nbands, fd_bpi, fd_segr, fd_rowsld;
};

static_assert(sizeof(StemBandArgs) <= 256, "kernel arguments fit one s_load batch");

template <int KB, int EPI>
__global__ void __launch_bounds__(64 * kSbWaves, 1) i8_stem_band_kernel(StemBandArgs a_in) {
  const StemBandArgs a = preload_args(a_in);
  // 4-byte outputs use natural channel order (MFMA row block j, row rho <-> channel 16j + rho),
  // so the 4 lanes of a pixel store 64 contiguous bytes per instruction; int8 outputs keep 16
  // consecutive channels per lane (one 16-byte store).
  constexpr bool NAT = EPI != kEpiI8;
  extern __shared__ v4i sb_lds[];
  const unsigned char* bytes = reinterpret_cast<const unsigned char*>(sb_lds);
  v4i* filt = sb_lds + a.filt_lds / 16;
  v4i* halo = sb_lds + a.halo_lds / 16;
  v4i* ep = sb_lds + a.ep_lds / 16;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row_l = lane & 15;
  const int grp_l = lane >> 4;

  const int lin = xcd_tile(blockIdx.x, a.nblocks);
  const int ctile = fdiv(lin, a.fd_nbands);
  const int band = lin - ctile * a.nbands;
  const int n = fdiv(band, a.fd_bpi);
  const int bi = band - n * a.bands_per_img;
  const int k0 = ctile * 64;
  const int ho0 = bi * a.BH;
  const int band_rows = min(a.BH, a.Ho - ho0);

  // ---- loads.  Filter instruction f (lane l: bytes [1024f + 16l, +16) of the tile's
  // 64 * RSC filter bytes, contiguous in KRSC) and input instruction i = row * rows_ld + m
  // go to wave f % 8 and i % 8; bias and scales to wave 0.
  {
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(k0) * a.RSC, 64 * a.RSC);
    for (int f = wave; f < a.nfilt; f += kSbWaves) load_lds16(rw, filt + f * 64, 16u * lane, 1024u * f);
  }
  if (EPI != kEpiAcc32 && wave == 0) {
    load_lds16(make_rsrc(a.bias ? a.bias + k0 : nullptr, a.bias ? 256 : 0), ep, 16u * lane, 0);
    load_lds16(make_rsrc(a.wscale + k0, 256), ep + 64, 16u * lane, 0);
  }
  {
    const int rowb = a.W * a.C;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + static_cast<size_t>(n) * a.H * rowb, a.H * rowb);
    const int hi0 = ho0 * a.sh - a.ph;
    const int ni = a.HR * a.rows_ld;
    for (int i = wave; i < ni; i += kSbWaves) {
      const int hr = fdiv(i, a.fd_rowsld);
      const int m = i - hr * a.rows_ld;
      const int hi = hi0 + hr;
      const int b = 1024 * m + 16 * lane - a.PLB;  // this lane's first byte in the input row
      const unsigned soff =
          static_cast<unsigned>(hi) < static_cast<unsigned>(a.H) ? static_cast<unsigned>(hi * rowb) : 0x40000000u;
      const unsigned voff = (b >= 0 && b + 16 <= rowb) ? static_cast<unsigned>(b) : 0x40000000u;
      load_lds16(rx, halo + i * 64, voff, soff);
    }
  }
  wait_vmcnt(0);
  barrier_only();

  // ---- filter fragments: lane (row_l, grp_l) of fragment (b, j) holds channel
  // 16*(row_l/4) + 4j + row_l%4 of the tile (natural order: 16j + row_l), chunk q = 4b + grp_l
  // (filter row q / CPR, bytes 16 * (q % CPR) .. of its SC-byte slot; bytes past SC and
  // chunks past NQ are 0).  The workgroup assembles each (channel, chunk) operand once from
  // the contiguous filter bytes into 16-byte slots, channel kl's chunk q at slot
  // 16 kl + ((q + kl + 4 (kl / 16)) mod 16): the 16 lanes of a lane group then read 16
  // distinct slots modulo 16 in either channel order.  Every wave then reads its fragments
  // with 16-byte LDS reads (assembled per wave instead, from five dwords and a funnel shift
  // each, the register copy took about 1 us on C5).
  const unsigned char* fbytes = bytes + a.filt_lds;
  v4i* slots = sb_lds + a.slot_lds / 16;
  auto slot_of = [](int kl, int q) { return 16 * kl + ((q + kl + 4 * (kl >> 4)) & 15); };
  for (int idx = threadIdx.x; idx < 64 * 4 * KB; idx += 64 * kSbWaves) {
    const int kl = idx / (4 * KB);
    const int q = idx - kl * (4 * KB);
    const int r = a.CPR == 2 ? (q >> 1) : q;
    const int h = q - r * a.CPR;
    const int nvalid = q < a.NQ ? min(16, a.SC - 16 * h) : 0;
    v4i v = lds_load16_unaligned(fbytes, kl * a.RSC + (nvalid > 0 ? r * a.SC + 16 * h : 0));
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int keep = min(4, max(0, nvalid - 4 * d));
      const unsigned msk = keep >= 4 ? 0xffffffffu : ((1u << (8 * keep)) - 1u);
      v[d] = static_cast<int>(static_cast<unsigned>(v[d]) & msk);
    }
    slots[slot_of(kl, q)] = v;
  }
  __syncthreads();
  v4i A[KB][4];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kl = NAT ? 16 * j + row_l : 16 * (row_l >> 2) + 4 * j + (row_l & 3);
      A[b][j] = slots[slot_of(kl, 4 * b + grp_l)];
    }
  }
  // epilogue parameters of this lane's 16 channels k0 + 16 * grp_l + 4j + r (natural order:
  // k0 + 16j + 4 * grp_l + r)
  v4i bias_v[4];
  v4f mult_v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bias_v[j] = v4i{0, 0, 0, 0};
    mult_v[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EPI != kEpiAcc32) {
      const int ev = NAT ? 4 * j + grp_l : 4 * grp_l + j;
      bias_v[j] = ep[ev];
      const v4i ws = ep[64 + ev];
#pragma unroll
      for (int r = 0; r < 4; ++r) mult_v[j][r] = requant_multiplier(a.act_scale, __int_as_float(ws[r]));
    }
  }
  // per K-block: byte offset of this lane's chunk within a staged band row window
  int qoff[KB];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    const int q = min(4 * b + grp_l, a.NQ - 1);  // chunks past NQ meet zero filter bytes
    const int r = a.CPR == 2 ? (q >> 1) : q;
    qoff[b] = r * a.dh * a.P + 16 * (q - r * a.CPR);
  }
  const float lo = a.relu ? 0.0f : -128.0f;
  constexpr int kOutBytes = EPI == kEpiI8 ? 1 : 4;
  const size_t out0 = (static_cast<size_t>(n) * a.Ho + ho0) * a.Wo * a.K + k0;
  const __amdgpu_buffer_rsrc_t ry =
      make_rsrc(static_cast<char*>(a.y) + out0 * kOutBytes, band_rows * a.Wo * a.K * kOutBytes);
  const unsigned char* hbytes = bytes + a.halo_lds;

  // A segment's operands: this lane's window starts at byte `base` of the band's staged
  // rows; K-block b's chunk lies qoff[b] further (a multiple of 16), so all of a segment's
  // reads share one dword alignment.  The five dwords of every chunk are read one segment
  // ahead, into `raw`, and funnel-shifted when the segment starts.
  const int nseg = band_rows * a.SEGR;
  auto window = [&](int sg, int& t, int& wo) {
    t = fdiv(sg, a.fd_segr);
    wo = 16 * (sg - t * a.SEGR) + row_l;
    return t * a.sh * a.P + a.PLB + ((wo < a.Wo ? wo : a.Wo - 1) * a.sw - a.pw) * a.C;
  };
  unsigned raw[KB][5];
  auto fetch = [&](int base) {
    const unsigned* p = reinterpret_cast<const unsigned*>(hbytes + (base & ~3));
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
      for (int i = 0; i < 5; ++i) raw[b][i] = p[qoff[b] / 4 + i];
  };
  int t = 0, wo = 0, base = 0;
  if (wave < nseg) {
    base = window(wave, t, wo);
    fetch(base);
  }
  for (int sg = wave; sg < nseg; sg += kSbWaves) {
    const unsigned sh = static_cast<unsigned>(base & 3);
    v4i B[KB];
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) B[b][i] = static_cast<int>(__builtin_amdgcn_alignbyte(raw[b][i + 1], raw[b][i], sh));
    const int t_cur = t, wo_cur = wo;
    // the next segment's reads may not move above the shifts that consume `raw`
    __builtin_amdgcn_sched_barrier(0);
    // (the last segment re-reads its own window: unconditional reads keep `raw` in place)
    base = window(sg + kSbWaves < nseg ? sg + kSbWaves : sg, t, wo);
    fetch(base);
    // a pixel past the row's end gets an offset 2^30 higher: past num_records, dropped
    const unsigned voff = static_cast<unsigned>(((t_cur * a.Wo + wo_cur) * a.K + (NAT ? 4 : 16) * grp_l) * kOutBytes) +
                          (static_cast<unsigned>(wo_cur >= a.Wo) << 30);
    v4i acc[4];
#pragma unroll
    for (int b = 0; b < KB; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b], b == 0 ? bias_v[j] : acc[j], 0, 0, 0);
    }
    if constexpr (EPI == kEpiI8) {
      const v4i pk = a.relu ? pack_u8_relu(acc, mult_v) : pack_i8(acc, mult_v, lo);
      __builtin_amdgcn_raw_buffer_store_b128(pk, ry, voff, 0, kStoreAux);
      store_gap(pk);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v4i v = acc[j];
        if constexpr (EPI == kEpiF32) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float f = static_cast<float>(acc[j][r]) * mult_v[j][r];
            if (a.relu) f = (f > 0.0f) ? f : 0.0f;  // NaN and -0 -> +0
            v[r] = __float_as_int(f);
          }
        }
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, voff + (NAT ? 64 : 16) * j, 0, kStoreAux);
        store_gap(v);
      }
    }
  }
}

struct StemBandPlan {
  int CPR, NQ, KB, BH, bands_per_img, HR, P, PLB, rows_ld, nfilt;
  int filt_lds, ep_lds, halo_lds;
  size_t lds;
};

int sb_cu_count() {
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

// The band variant needs what the general stem kernel needs plus: whole 16-byte chunks
// per input row (W*C % 16 == 0, so no load straddles a row end), whole 64-channel tiles
// (K % 64 == 0: filter slice, bias and scales in whole loads) and its rows in LDS.
bool make_band_plan(const Geom& g, StemBandPlan* pl) {
  const int SC = g.S * g.C;
  pl->CPR = SC <= 16 ? 1 : 2;
  pl->NQ = g.R * pl->CPR;
  pl->KB = (pl->NQ + 3) / 4;
  if (pl->KB > 4 || g.dw != 1) return false;
  const long long rowb = static_cast<long long>(g.W) * g.C;
  if (rowb % 16 != 0 || g.K % 64 != 0) return false;
  if (static_cast<long long>(g.H) * rowb >= (1LL << 30)) return false;
  if (static_cast<long long>(g.Ho) * g.Wo * g.K * 4 >= (1LL << 30)) return false;
  pl->PLB = round_up(std::max(0, g.pw) * g.C, 16);
  // last byte any lane reads in a staged row: window of the last output column, its
  // row slot and the 4-byte over-read of the unaligned LDS loader
  const long long last = pl->PLB + (static_cast<long long>(g.Wo - 1) * g.sw - g.pw) * g.C + 16LL * pl->CPR + 4;
  const long long need = std::max<long long>(pl->PLB + rowb, last);
  pl->P = static_cast<int>((need + 1023) / 1024 * 1024);
  pl->rows_ld = pl->P / 1024;
  const long long RSC = static_cast<long long>(g.R) * SC;
  pl->nfilt = static_cast<int>((64 * RSC + 20 + 1023) / 1024);  // + the loader's over-read
  const int segr = (g.Wo + 15) / 16;
  const int cus = sb_cu_count();
  // filter, then 2 KB for bias and scales (each of their two loads writes all 64 lanes) and
  // 16 KB of filter operand slots (64 channels x 16 chunks)
  const size_t fixed = static_cast<size_t>(pl->nfilt) * 1024 + 2048 + 16384;
  bool found = false;
  double best = 0.0;
  for (int bh = 1; bh <= g.Ho; ++bh) {
    const long long hr = static_cast<long long>(bh - 1) * g.sh + static_cast<long long>(g.R - 1) * g.dh + 1;
    const size_t lds = fixed + static_cast<size_t>(hr) * pl->P;
    if (lds > static_cast<size_t>(kSbLds)) break;
    const long long bands = (g.Ho + bh - 1) / bh;
    const long long wgs = static_cast<long long>(g.N) * bands * (g.K / 64);
    const long long rounds = (wgs + cus - 1) / cus;
    // segments per wave plus a fixed cost for the loads
    const double cost = static_cast<double>(rounds) * ((bh * segr + kSbWaves - 1) / kSbWaves + 3);
    if (!found || cost < best - 1e-9) {
      found = true;
      best = cost;
      pl->BH = bh;
      pl->bands_per_img = static_cast<int>(bands);
      pl->HR = static_cast<int>(hr);
      pl->filt_lds = 0;
      pl->ep_lds = pl->nfilt * 1024;
      pl->halo_lds = pl->ep_lds + 2048 + 16384;
      pl->lds = lds;
    }
  }
  if (!found) return false;
  const long long blocks = static_cast<long long>(g.N) * pl->bands_per_img * (g.K / 64);
  return blocks <= 0x7fffffffLL;
}

template <int EPI>
void launch_band(const StemBandArgs& a, const StemBandPlan& pl, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.nblocks));
  auto go = [&](auto kern) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(pl.lds));
    hipLaunchKernelGGL(kern, grid, dim3(64 * kSbWaves), pl.lds, stream, a);
  };
  switch (pl.KB) {
    case 1: go(i8_stem_band_kernel<1, EPI>); break;
    case 2: go(i8_stem_band_kernel<2, EPI>); break;
    case 3: go(i8_stem_band_kernel<3, EPI>); break;
    default: go(i8_stem_band_kernel<4, EPI>); break;
  }
}

hipError_t launch_stem_band(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                            const StemBandPlan& pl, hipStream_t stream) {
  StemBandArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = y;
  a.H = g.H; a.W = g.W; a.C = g.C; a.K = g.K; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.sh = g.sh; a.sw = g.sw; a.dh = g.dh;
  a.SC = g.S * g.C; a.RSC = g.R * a.SC; a.CPR = pl.CPR; a.NQ = pl.NQ;
  a.BH = pl.BH; a.bands_per_img = pl.bands_per_img; a.nbands = g.N * pl.bands_per_img;
  a.nblocks = a.nbands * (g.K / 64);
  a.SEGR = (g.Wo + 15) / 16;
  a.P = pl.P; a.PLB = pl.PLB; a.rows_ld = pl.rows_ld; a.HR = pl.HR; a.nfilt = pl.nfilt;
  a.filt_lds = pl.filt_lds; a.ep_lds = pl.ep_lds; a.halo_lds = pl.halo_lds; a.slot_lds = pl.ep_lds + 2048;
  a.act_scale = rq.act_scale; a.relu = rq.relu;
  a.fd_nbands = fastdiv_m(a.nbands);
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_segr = fastdiv_m(a.SEGR);
  a.fd_rowsld = fastdiv_m(pl.rows_ld);
  switch (epi) {
    case kEpiI8: launch_band<kEpiI8>(a, pl, stream); break;
    case kEpiAcc32: launch_band<kEpiAcc32>(a, pl, stream); break;
    default: launch_band<kEpiF32>(a, pl, stream); break;
  }
  return hipGetLastError();
}

struct StemPlan {
  int RowB, CPR, NQ, KB;
  int RB, tiles_h;
  int PL, P, w_off, w_bytes, ep_off;
  size_t lds;
};

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
  {
    StemBandPlan bp;
    if (make_band_plan(g, &bp)) return launch_stem_band(g, epi, x, w, y, rq, bp, stream);
  }
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
