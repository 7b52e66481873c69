// int8 convolution for 64 -> 64-channel stride-1 layers with an odd number of taps (ResNet
// conv2_x 3x3): a row band per workgroup whose input rows stream into LDS while the matrix
// instructions run, filter-stationary v_mfma_i32_16x16x64_i8, fused bias / requantize / ReLU /
// int8 saturate.
//
// Work.  A workgroup owns a band of BH output rows of one image, all 64 output channels.  Its
// bh * Wo output pixels are numbered row-major (q = t * Wo + c) and cut into 16-pixel segments
// that run on across row ends, so only the band's last segment is partly empty.  Eight compute
// waves: wave w (on SIMD w % 4) computes the 32 channels 32h .. 32h + 31 (h = w & 1) of the
// segment pairs (2P, 2P + 1) with P = m, m + 4, m + 8, ... (m = w >> 1).  Per K-block a pair is
// two B fragments and four independent accumulator chains, and each SIMD carries the same
// number of segments to within one (ResNet-50 3x3, 7 rows: 13, 13, 12, 12, against the 14 or
// 16 row-aligned segments per SIMD of a wave-per-64-channels split).
//
// Loader waves.  Two more waves load the band's halo rows (global -> LDS DMA, no registers),
// rows l, l + 2, ... for loader l: first the rows the first segment pairs read, alone, then the
// rest, all before any output store of the workgroup is issued.  Loads complete in order, so a
// loader publishes the count of its rows landed in an LDS word after each compile-time
// s_waitcnt of a fully unrolled descending sequence.  A compute wave waits on the two counts
// (s_sleep polling, bounded) for the rows its next pair reads.  The filter is loaded by the
// compute waves; each counts its share landed, and every wave starts once all eight have.
// Counts are zeroed before one barrier at entry; nothing else synchronises with a barrier.
//
// Input rows in LDS.  Halo row hr (input row ho0 - ph + hr) is a virtual row of RowS pixels
// (RowS >= 16 * NJ >= Wo + (S-1)*dw, RowS = Wo mod 16), halo pixel p = hr * RowS + col holds
// input column col - pw, zero outside the image.  Output pixel q = t * Wo + c reads, for tap
// (r, s), halo pixel p = (t + r*dh) * RowS + c + s*dw; because RowS = Wo (mod 16), the 16
// pixels of a segment are 16 consecutive values of p modulo 16 even where the segment crosses
// a row end.  Pixel p's four 16-channel chunks sit at 16-byte slots 4p + (chunk ^ f(p)), f(p) =
// 2 * ((p >> 2) & 1): a ds_read_b128 of 16 pixels x one chunk per lane group meets 16 distinct
// slots modulo 16 in each of its four cycles (the measured bank rule: a cycle serves one
// half-wave's lane quads of equal bit parity).  A 1 KB DMA instruction covers 16 consecutive
// halo pixels of one row (NJ per row), each pixel's 64 bytes read by four lanes.
//
// Filter in LDS.  The 64 KRSC rows (64 * Kdim bytes) are loaded as they lie, 1 KB per
// instruction, with the 16-byte units of channel k at slots 4KB*k + (u ^ 2*((k >> 3) & 1)): the
// swap of unit pairs in channels 8..15 mod 16 makes every A-fragment read conflict-free (odd
// KB).  Each compute wave copies its 32 channels (KB x 2 fragments) into registers once.
// MFMA row rho of tile j is channel 32h + 8*(rho/4) + 4j + rho%4, so an output lane holds 8
// consecutive channels of one pixel.
//
// Output.  Accumulators start at the bias; convert, scale, clamp and round to nearest even
// exactly as the other int8 kernels (clamp to [lo, 127], the 1.5 * 2^23 addition, bytes
// packed with v_perm_b32).  A wave writes its 32 channels of a segment into an LDS staging area (96 bytes per
// pixel) and counts the half staged; the wave that stages the second half stores the whole
// segment (16 pixels x 64 channels, one contiguous kilobyte of NHWC output) with one 16-byte
// write-through non-temporal store per lane, followed by store_gap() on its data registers.
// Compute waves issue no global load after the filter, so no vector-memory wait of theirs ever
// waits for a store.

#include "qconv_device.h"

#include <algorithm>
#include <type_traits>

namespace miq {
namespace {

constexpr int kPipeCompute = 8;                 // compute waves (two per SIMD)
constexpr int kPipeLoaders = 2;                 // loader waves: halo rows l, l + 2, ...
constexpr int kPipeWaves = kPipeCompute + kPipeLoaders;
constexpr int kPipeLds = 160 * 1024;
constexpr int kPipeMaxNJ = 8;                   // load instructions per halo row (16 pixels each)
// LDS byte offsets: the loaders' rows-landed counts and the filter-landed count; bias
// int32[64] at kPipeEp and scales f32[64] at kPipeEp + 1024 (each loaded by one 1 KB DMA
// instruction whose lanes past the 64 values write zeros); the filter (64 * Kdim bytes); then
// the halo
constexpr int kPipeFlag = 1024;
constexpr int kPipeSegCount = 1088;             // staged halves per segment (one word each)
constexpr int kPipeMaxSeg = (2048 - kPipeSegCount) / 4;
constexpr unsigned kPipeStagePx = 96;                  // LDS bytes per staged output pixel (64 used)
constexpr unsigned kPipeStageSeg = 16 * kPipeStagePx;  // per staged segment of 16 pixels
constexpr int kPipeEp = 2048;
constexpr int kPipeFilt = 4096;

__host__ __device__ constexpr int pipe_halo_lds(int KB) { return kPipeFilt + 64 * 64 * KB; }

struct PipeArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  int8_t* y;
  int H, W, Ho, Wo;
  int ph, pw, dh, dw;
  int BH;             // output rows per band
  int bands_per_img;  // ceil(Ho / BH)
  int nblocks;        // workgroups of the launch
  int RowS;           // virtual halo row length (pixels)
  int HR;             // halo rows per band: BH + (R-1)*dh
  int NJ;             // load instructions per halo row: ceil(cols / 16)
  int cols;           // halo columns read: Wo + (S-1)*dw
  int rows0;          // halo rows the first segment pairs (segments 0 .. 7) read: loaded first
  int out_lds;        // LDS byte offset of the output staging area (1 KB per segment)
  int rstep;          // LDS bytes between tap rows: dh * RowS * 64
  float act_scale;
  FastDivM fd_bpi, fd_wo;
};

static_assert(sizeof(PipeArgs) <= 256, "kernel arguments fit one s_load batch");

__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>(p) & 0xffffffffu);
}

// 8 requantized outputs of one lane (channels 4j + i of its 8, j = 0, 1) as two packed dwords.
template <bool RELU>
__device__ __forceinline__ void pack8(const v4i& a0, const v4i& a1, const v4f (&m)[2], unsigned& d0, unsigned& d1) {
  const float lo = RELU ? 0.0f : -128.0f;
  float c[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = requant_magic(a0[i], m[0][i], lo);
    c[4 + i] = requant_magic(a1[i], m[1][i], lo);
  }
  d0 = pack4_magic(c[0], c[1], c[2], c[3]);
  d1 = pack4_magic(c[4], c[5], c[6], c[7]);
}

// s_waitcnt vmcnt(n) for a compile-time 0 <= n <= 63 (bits 3:0 and 15:14 of the immediate).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0xF70 | (N & 15) | ((N >> 4) << 14));
}

// Loader wave l: halo rows l, l + kPipeLoaders, ... of the band (K of them), NJ load
// instructions each (instruction (hr, j) covers halo pixels hr * RowS + 16j .. + 15 and never
// crosses a row, since 16 * NJ <= RowS), all issued at entry so that they queue ahead of every
// output store of the workgroup.  Loads complete in order, so its k-th row has landed once
// vmcnt <= (K - 1 - k) * NJ; the waits run down a fully unrolled sequence of compile-time
// s_waitcnt steps (one uniform branch each, no branch tree), each followed by publishing the
// count of this loader's rows landed.  Lane l reads column 16j + l/4, chunk (l % 4) ^ f(p),
// f(p) depending on bit 2 of l/4 only (RowS and 16j are multiples of 8): the lane's offset
// within a row is one of NJ loop-invariant values.
// The waits of a loader with K rows in flight, from vmcnt <= (K - 1) * NJ down to 0: step M
// (M = MMAX, MMAX - 1, ..., 0) runs when M < K and publishes K - M landed rows.
template <int NJ, int M>
__device__ __forceinline__ void loader_publish(int K, int done, int* myflag, int lane) {
  if constexpr (M >= 0) {
    if (M < K) {
      wait_vm<M * NJ>();
      asm volatile("" ::: "memory");
      if (lane == 0) lds_publish(myflag, done + K - M);
    }
    loader_publish<NJ, M - 1>(K, done, myflag, lane);
  }
}

template <int NJ>
__device__ __forceinline__ void pipe_loader(const PipeArgs& a, unsigned halo_b, int n, int ho0, int* myflag, int l,
                                            int lane) {
  constexpr int kMaxRows = 63 / NJ;  // rows per loader within the vmcnt range
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + static_cast<size_t>(n) * a.H * a.W * 64, a.H * a.W * 64);
  const int hi0 = ho0 - a.ph;
  const int lp = lane >> 2;
  const unsigned ch16 = 16u * static_cast<unsigned>((lane & 3) ^ ((lp >> 1) & 2));
  unsigned vj[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = 16 * j + lp;
    const int wi = col - a.pw;
    const bool ok = col < a.cols && static_cast<unsigned>(wi) < static_cast<unsigned>(a.W);
    vj[j] = ok ? static_cast<unsigned>(wi) * 64u + ch16 : 0x40000000u;
  }
  auto issue_row = [&](int hr) {
    const int hi = hi0 + hr;
    // an image row outside the image: every lane past num_records (reads zeros)
    const bool row_ok = static_cast<unsigned>(hi) < static_cast<unsigned>(a.H);
    const unsigned soff = row_ok ? static_cast<unsigned>(hi * a.W) * 64u : 0u;
    const unsigned row_lds = halo_b + static_cast<unsigned>(hr * a.RowS) * 64u;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const unsigned voff = row_ok ? vj[j] : 0x40000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(static_cast<uintptr_t>(row_lds + 1024u * j)), 16, voff,
                                               soff, 0, 0);
    }
  };
  // First the rows the wave's first segment pairs read (halo rows below a.rows0), alone, so
  // that they are not queued behind the rest of the band's loads of every CU; then the rest.
  int K0 = 0, K = 0;
  int hr = l;
  for (; hr < a.rows0; hr += kPipeLoaders, ++K0) issue_row(hr);
  loader_publish<NJ, kMaxRows - 1>(K0, 0, myflag, lane);
  for (; hr < a.HR; hr += kPipeLoaders, ++K) issue_row(hr);
  // the k-th row has landed once vmcnt <= (K - 1 - k) * NJ
  loader_publish<NJ, kMaxRows - 1>(K, K0, myflag, lane);
}

template <int R, int S, bool RELU>
__global__ void __launch_bounds__(64 * kPipeWaves, 1) i8_pipe_kernel(PipeArgs a_in) {
  constexpr int KB = R * S;  // one 64-deep K-block per tap (64 input channels)
  static_assert((KB & 1) == 1 && KB <= 9, "odd tap count, filter in registers");
  constexpr int kHalo = pipe_halo_lds(KB);
  const PipeArgs a = preload_args(a_in);
  extern __shared__ v4i smem[];
  const unsigned base = lds_addr(smem);
  // The rows-landed word is read and written with relaxed workgroup-scope atomics: plain LDS
  // accesses that the compiler neither caches in a register nor surrounds with the
  // vector-memory waits a volatile access gets (which would wait for this wave's stores).
  int* flag = reinterpret_cast<int*>(reinterpret_cast<char*>(smem) + kPipeFlag);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const int band = xcd_tile(blockIdx.x, a.nblocks);
  const int n = fdiv(band, a.fd_bpi);
  const int ho0 = (band - n * a.bands_per_img) * a.BH;
  const int bh = min(a.BH, a.Ho - ho0);
  const int band_px = bh * a.Wo;

  // The zeroed counts are published by a barrier at entry, before any wave reads or adds to
  // them; no wave synchronises with a barrier after that.
  // flag[l]: rows of loader l landed; flag[kPipeLoaders]: compute waves whose share of the
  // filter has landed
  int* fcount = flag + kPipeLoaders;
  // scount[s]: halves (32-channel parts) of output segment s staged in LDS
  int* scount = reinterpret_cast<int*>(reinterpret_cast<char*>(smem) + kPipeSegCount);
  if (wave >= kPipeCompute) {
    if (lane == 0) {
      __hip_atomic_store(flag + (wave - kPipeCompute), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (wave == kPipeCompute) __hip_atomic_store(fcount, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    for (int c = (wave - kPipeCompute) * 64 + lane; c < kPipeMaxSeg; c += 64 * kPipeLoaders)
      __hip_atomic_store(scount + c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  barrier_only();

  if (wave >= kPipeCompute) {
    const unsigned halo_b = base + kHalo;
    const int l = wave - kPipeCompute;
    int* myflag = flag + l;
    switch (a.NJ) {
      case 1: pipe_loader<1>(a, halo_b, n, ho0, myflag, l, lane); break;
      case 2: pipe_loader<2>(a, halo_b, n, ho0, myflag, l, lane); break;
      case 3: pipe_loader<3>(a, halo_b, n, ho0, myflag, l, lane); break;
      case 4: pipe_loader<4>(a, halo_b, n, ho0, myflag, l, lane); break;
      case 5: pipe_loader<5>(a, halo_b, n, ho0, myflag, l, lane); break;
      case 6: pipe_loader<6>(a, halo_b, n, ho0, myflag, l, lane); break;
      case 7: pipe_loader<7>(a, halo_b, n, ho0, myflag, l, lane); break;
      default: pipe_loader<8>(a, halo_b, n, ho0, myflag, l, lane); break;
    }
    return;
  }

  // ---- compute waves: the filter (and bias, scales) into LDS, spread over the 8 waves ----
  {
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, 64 * 64 * KB);
    // instruction i: slot 64i + lane = channel k, unit u' -> global unit u' ^ 2*((k >> 3) & 1)
    for (int i = wave; i < 4 * KB; i += kPipeCompute) {
      const int slot = 64 * i + lane;
      const int k = slot / (4 * KB);
      const int u = (slot - k * 4 * KB) ^ ((k >> 2) & 2);
      load_lds16(rw, smem + kPipeFilt / 16 + 64 * i, static_cast<unsigned>(k * 64 * KB + 16 * u), 0);
    }
    if (wave == kPipeCompute - 2) {
      load_lds16(make_rsrc(a.bias, a.bias ? 256 : 0), smem + kPipeEp / 16, 16u * lane, 0);
    } else if (wave == kPipeCompute - 1) {
      load_lds16(make_rsrc(a.wscale, 256), smem + (kPipeEp + 1024) / 16, 16u * lane, 0);
    }
  }
  wait_vmcnt(0);
  if (lane == 0) __hip_atomic_fetch_add(fcount, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  // bounded: every compute wave adds once, so this ends long before the bound
  for (int it = 0; it < (1 << 20); ++it) {
    if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(fcount, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) >=
        kPipeCompute)
      break;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");

  const int h = wave & 1;   // channel half
  const int m = wave >> 1;  // segment-pair class
  const int rho = lane & 15;
  const int g = lane >> 4;

  // The filter in registers: A[b][j], lane (rho, g) = channel 32h + 8*(rho/4) + 4j + rho%4,
  // bytes [64b + 16g, +16) of its row.
  v4i A[KB][2];
  {
    const int kc = 32 * h + 8 * (rho >> 2) + (rho & 3);
    const unsigned sw = static_cast<unsigned>(g ^ ((rho >> 1) & 2));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const unsigned fa = base + kPipeFilt + 64u * KB * static_cast<unsigned>(kc + 4 * j) + 16u * sw;
#pragma unroll
      for (int b = 0; b < KB; ++b) A[b][j] = lds_read16(fa + 64u * b);
    }
  }
  // bias and requantization multipliers of the lane's output channels 32h + 8g + 4j + i
  v4i bias_v[2];
  v4f mult_v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const unsigned ca = base + kPipeEp + 4u * static_cast<unsigned>(32 * h + 8 * g + 4 * j);
    bias_v[j] = lds_read16(ca);
    const v4i ws = lds_read16(ca + 1024u);
#pragma unroll
    for (int i = 0; i < 4; ++i) mult_v[j][i] = requant_multiplier(a.act_scale, __int_as_float(ws[i]));
  }

  const int nseg = (band_px + 15) >> 4;
  const unsigned g16 = 16u * static_cast<unsigned>(g);
  const unsigned halo = base + kHalo;
  // this lane's 8 output bytes of segment seg in the LDS staging area: pixel rho, channels
  // 32h + 8g .. + 7.  A staged pixel takes kPipeStagePx bytes: the 8-byte writes of a wave
  // meet each bank at most twice, and the 16-byte reads of a whole segment (lane l: pixel
  // l % 16, channels 16 * (l / 16) ..) are free of bank conflicts.
  const unsigned stage_lane = base + static_cast<unsigned>(a.out_lds) + kPipeStagePx * rho + 32u * h + 8u * g;

  // LDS byte address of this lane's B fragment of segment `seg`, tap column s (tap row r adds
  // r * rstep)
  auto seg_addr = [&](int seg, unsigned (&ad)[S]) {
    const int q = min(16 * seg + rho, band_px - 1);
    const int t = fdiv(q, a.fd_wo);
    const int p = t * a.RowS + q - t * a.Wo;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const unsigned ps = static_cast<unsigned>(p + s * a.dw);
      ad[s] = halo + (((ps << 6) | g16) ^ ((ps << 3) & 32u));
    }
  };
  int seen = 0;  // rows known to have landed (wave-uniform)
  // rows 0 .. need-1 have landed once loader l has published (need - l + 1) / 2 of its rows
  static_assert(kPipeLoaders == 2, "one 8-byte read of both counts");
  auto wait_rows = [&](int need) {
    if (need <= seen) return;
    const int want0 = (need + 1) >> 1, want1 = need >> 1;
    // bounded: the loaders publish every row, so this ends long before the bound
    for (int it = 0; it < (1 << 20); ++it) {
      const long long both = __hip_atomic_load(reinterpret_cast<long long*>(flag), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
      const int c0 = __builtin_amdgcn_readfirstlane(static_cast<int>(both));
      const int c1 = __builtin_amdgcn_readfirstlane(static_cast<int>(both >> 32));
      if (c0 >= want0 && c1 >= want1) {
        seen = min(2 * c0, 2 * c1 + 1);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
  };
  // The requantized half-segment (32 channels) goes to the LDS staging area and the segment's
  // count of staged halves is raised (LDS operations of a wave complete in order, so a count
  // seen raised means its bytes are written).  The odd-half waves (h == 1) store whole segments
  // (16 pixels x 64 channels, one contiguous kilobyte of NHWC output, one 16-byte
  // write-through non-temporal store per lane): those of a pair once they have computed the
  // next pair, when the even-half wave of the same segments has staged its half as well.
  // Nothing in this waits on an atomic's return.
  const size_t out0 = (static_cast<size_t>(n) * a.Ho + ho0) * a.Wo * 64;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y + out0, band_px * 64);
  typedef int v2i __attribute__((ext_vector_type(2)));
  auto stage = [&](int seg, const v4i& a0, const v4i& a1) {
    unsigned d0, d1;
    pack8<RELU>(a0, a1, mult_v, d0, d1);
    *reinterpret_cast<__attribute__((address_space(3))) v2i*>(static_cast<uintptr_t>(stage_lane + kPipeStageSeg * seg)) =
        v2i{static_cast<int>(d0), static_cast<int>(d1)};
    if (lane == 0) __hip_atomic_fetch_add(scount + seg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  auto store_seg = [&](int seg) {
    const v4i d = lds_read16(base + static_cast<unsigned>(a.out_lds) + kPipeStageSeg * seg + kPipeStagePx * rho + 16u * g);
    // pixels past the band get an offset past num_records (dropped), in voffset itself
    const unsigned voff = 1024u * seg + 64u * rho + 16u * g + (16 * seg + rho < band_px ? 0u : 0x40000000u);
    __builtin_amdgcn_raw_buffer_store_b128(d, ry, voff, 0, kStoreAux);
    store_gap(d);
  };
  // segments ps and ps + 1 (when two) once both halves of each are staged (ps even: the two
  // counts are one aligned 8-byte word)
  auto store_pair = [&](int ps, bool two) {
    // bounded: the even-half wave stages every half, so this ends long before the bound
    for (int it = 0; it < (1 << 20); ++it) {
      const long long both = __hip_atomic_load(reinterpret_cast<long long*>(scount + ps), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
      const int c0 = __builtin_amdgcn_readfirstlane(static_cast<int>(both));
      const int c1 = __builtin_amdgcn_readfirstlane(static_cast<int>(both >> 32));
      if (c0 >= 2 && (!two || c1 >= 2)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
    store_seg(ps);
    if (two) store_seg(ps + 1);
  };
  int pend = -1;        // the odd-half wave's pair waiting to be stored (first segment), or -1
  bool pend_two = false;

  const int rext = (R - 1) * a.dh + 1;
  for (int pp = m; 2 * pp < nseg; pp += 4) {
    const int s0 = 2 * pp;
    const bool two = s0 + 1 < nseg;
    const int qlast = min(16 * s0 + (two ? 31 : 15), band_px - 1);
    wait_rows(min(a.HR, fdiv(qlast, a.fd_wo) + rext));
    unsigned ad0[S], ad1[S];
    seg_addr(s0, ad0);
    if (two) {
      seg_addr(s0 + 1, ad1);
      v4i c00, c01, c10, c11;
      constexpr int RS = KB < 2 ? KB : 2;
      v4i B0[RS], B1[RS];
#pragma unroll
      for (int b = 0; b < RS; ++b) {
        B0[b] = lds_read16(ad0[b % S] + static_cast<unsigned>(b / S) * a.rstep);
        B1[b] = lds_read16(ad1[b % S] + static_cast<unsigned>(b / S) * a.rstep);
      }
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        c00 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][0], B0[b % RS], b == 0 ? bias_v[0] : c00, 0, 0, 0);
        c10 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][0], B1[b % RS], b == 0 ? bias_v[0] : c10, 0, 0, 0);
        c01 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][1], B0[b % RS], b == 0 ? bias_v[1] : c01, 0, 0, 0);
        c11 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][1], B1[b % RS], b == 0 ? bias_v[1] : c11, 0, 0, 0);
        if (b + RS < KB) {
          const int bn = b + RS;
          B0[b % RS] = lds_read16(ad0[bn % S] + static_cast<unsigned>(bn / S) * a.rstep);
          B1[b % RS] = lds_read16(ad1[bn % S] + static_cast<unsigned>(bn / S) * a.rstep);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      stage(s0, c00, c01);
      stage(s0 + 1, c10, c11);
      if (h == 1 && pend >= 0) store_pair(pend, pend_two);
      pend = s0;
      pend_two = true;
    } else {
      v4i c00, c01;
      constexpr int RS = KB < 3 ? KB : 3;
      v4i B0[RS];
#pragma unroll
      for (int b = 0; b < RS; ++b) B0[b] = lds_read16(ad0[b % S] + static_cast<unsigned>(b / S) * a.rstep);
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        c00 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][0], B0[b % RS], b == 0 ? bias_v[0] : c00, 0, 0, 0);
        c01 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][1], B0[b % RS], b == 0 ? bias_v[1] : c01, 0, 0, 0);
        if (b + RS < KB) {
          const int bn = b + RS;
          B0[b % RS] = lds_read16(ad0[bn % S] + static_cast<unsigned>(bn / S) * a.rstep);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      stage(s0, c00, c01);
      if (h == 1 && pend >= 0) store_pair(pend, pend_two);
      pend = s0;
      pend_two = false;
    }
  }
  if (h == 1 && pend >= 0) store_pair(pend, pend_two);
}

struct PipePlan {
  int BH, bands_per_img, RowS, HR, NJ, cols;
  size_t lds_bytes;
};

int pipe_cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

bool pipe_plan(const Geom& g, Epi epi, PipePlan* p, std::string* why) {
  auto no = [&](const char* m) { if (why) *why = m; return false; };
  if (epi != kEpiI8) return no("pipe kernel writes int8 outputs only");
  if (g.G != 1 || g.C != 64 || g.K != 64) return no("pipe kernel needs groups == 1 and 64 input and output channels");
  if (g.sh != 1 || g.sw != 1) return no("pipe kernel needs stride 1");
  if (g.dh < 1 || g.dw < 1 || g.ph < 0 || g.pw < 0) return no("pipe kernel needs positive dilation");
  if (!((g.R == 3 && g.S == 3) || (g.R == 1 && g.S == 1))) return no("pipe kernel needs a 3x3 or 1x1 filter");
  if (g.Wo % 8 != 0) return no("pipe kernel needs output width % 8 == 0");
  if (static_cast<long long>(g.H) * g.W * 64 >= (1LL << 30)) return no("pipe kernel needs images below 2^30 bytes");
  if (static_cast<long long>(g.Ho) * g.Wo * 64 >= (1LL << 30)) return no("pipe kernel needs images below 2^30 output bytes");
  const long long cols = static_cast<long long>(g.Wo) + static_cast<long long>(g.S - 1) * g.dw;
  // NJ 16-pixel load instructions per halo row; the virtual row length RowS is the smallest
  // >= 16 * NJ with RowS = Wo (mod 16)
  const long long nj = (cols + 15) / 16;
  if (nj > kPipeMaxNJ) return no("pipe kernel needs output width + dilated filter width <= 128");
  const long long rows = 16 * nj + ((g.Wo - 16 * nj) % 16 + 16) % 16;
  const int KB = g.R * g.S;
  const int cus = pipe_cu_count();
  bool found = false;
  double best = 0.0;
  for (int bh = 1; bh <= g.Ho; ++bh) {
    const long long hr = bh + static_cast<long long>(g.R - 1) * g.dh;
    if (((hr + kPipeLoaders - 1) / kPipeLoaders) * nj > 63) break;  // one loader's loads within its vmcnt range
    const long long nseg = (static_cast<long long>(bh) * g.Wo + 15) / 16;
    if (nseg > kPipeMaxSeg) break;
    const size_t lds = static_cast<size_t>(pipe_halo_lds(KB)) + static_cast<size_t>(hr * rows) * 64 +
                       static_cast<size_t>(nseg) * kPipeStageSeg;
    if (lds > static_cast<size_t>(kPipeLds)) break;
    if (static_cast<long long>(g.R - 1) * g.dh * rows * 64 >= (1LL << 20)) break;
    const long long bands = (g.Ho + bh - 1) / bh;
    const long long wgs = static_cast<long long>(g.N) * bands;
    const long long rounds = (wgs + cus - 1) / cus;
    // the busiest SIMD: pair classes 0 and 2 (segments 0, 1 mod 8 and 4, 5 mod 8)
    long long simd_seg = 0;
    for (long long s = 0; s < nseg; ++s) simd_seg += ((s >> 1) & 1) == 0 ? 1 : 0;
    // cycles: one segment is 2 * KB matrix instructions of 16 cycles; start-up (loads of the
    // filter and the first rows) about 2000
    const double cost = static_cast<double>(rounds) * (2000.0 + static_cast<double>(simd_seg) * KB * 32.0);
    if (!found || cost < best - 1e-9) {
      found = true;
      best = cost;
      p->BH = bh;
      p->bands_per_img = static_cast<int>(bands);
      p->RowS = static_cast<int>(rows);
      p->HR = static_cast<int>(hr);
      p->NJ = static_cast<int>(nj);
      p->cols = static_cast<int>(cols);
      p->lds_bytes = lds;
    }
  }
  if (!found) return no("pipe kernel input rows do not fit its loads");
  if (static_cast<long long>(g.N) * p->bands_per_img > 0x7fffffffLL) return no("grid too large");
  return true;
}

template <int R, int S>
void pipe_launch_rs(const PipeArgs& a, const PipePlan& pl, int relu, unsigned nblocks, hipStream_t stream) {
  auto kern = relu ? i8_pipe_kernel<R, S, true> : i8_pipe_kernel<R, S, false>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(pl.lds_bytes));
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(64 * kPipeWaves), pl.lds_bytes, stream, a);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool pipe_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                   std::string* why) {
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || (rq.bias != nullptr && !aligned16(rq.bias)) ||
      !aligned16(rq.wscale)) {
    if (why) *why = "pipe kernel needs 16-byte aligned tensors, bias and scales";
    return false;
  }
  PipePlan pl;
  return pipe_plan(g, epi, &pl, why);
}

hipError_t launch_i8_pipe(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream) {
  if (static_cast<long long>(g.N) * g.Ho * g.Wo * g.K == 0) return hipSuccess;
  PipePlan pl;
  if (!pipe_plan(g, epi, &pl, nullptr)) return hipErrorInvalidConfiguration;
  PipeArgs a;
  a.x = x; a.w = w; a.bias = rq.bias; a.wscale = rq.wscale; a.y = static_cast<int8_t*>(y);
  a.H = g.H; a.W = g.W; a.Ho = g.Ho; a.Wo = g.Wo;
  a.ph = g.ph; a.pw = g.pw; a.dh = g.dh; a.dw = g.dw;
  a.BH = pl.BH; a.bands_per_img = pl.bands_per_img;
  a.RowS = pl.RowS; a.HR = pl.HR; a.NJ = pl.NJ; a.cols = pl.cols;
  a.rstep = g.dh * pl.RowS * 64;
  a.out_lds = pipe_halo_lds(g.R * g.S) + pl.HR * pl.RowS * 64;
  a.rows0 = std::min(pl.HR, (std::min(127, std::min(pl.BH, g.Ho) * g.Wo - 1)) / g.Wo + (g.R - 1) * g.dh + 1);
  a.act_scale = rq.act_scale;
  a.fd_bpi = fastdiv_m(pl.bands_per_img);
  a.fd_wo = fastdiv_m(g.Wo);
  const long long nblocks = static_cast<long long>(g.N) * pl.bands_per_img;
  a.nblocks = static_cast<int>(nblocks);
  if (g.R == 3) {
    pipe_launch_rs<3, 3>(a, pl, rq.relu, static_cast<unsigned>(nblocks), stream);
  } else {
    pipe_launch_rs<1, 1>(a, pl, rq.relu, static_cast<unsigned>(nblocks), stream);
  }
  return hipGetLastError();
}

}  // namespace miq
