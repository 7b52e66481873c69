// int8 pointwise (1x1, stride 1, no padding) convolution with 64 or 128 input channels:
// a GEMM over the flattened output pixels (P = n*h*w, each pixel's C input bytes contiguous in
// NHWC), filter-stationary v_mfma_i32_16x16x64_i8, with the input streamed into LDS by four
// loader waves while eight compute waves consume it.
//
// Work.  The P pixels are cut into 16-pixel segments; the segments are split into contiguous
// ranges.  A workgroup owns one range and NT (1 or 2) 64-channel output tiles: NT*64 channels.
// The workgroups of one range (one per channel-tile group) are launched on the same XCD, so the
// range's input comes from HBM once and from that XCD's L2 after.  Compute wave w takes tile
// t = w % NT and every (8/NT)-th segment of the range from w / NT on; per segment it runs
// KB x 4 MFMAs (KB = C/64 K-blocks, 4 row blocks of 16 channels), requantizes the 16 x 64
// result (16 channels of one pixel per lane) and stores it with one 16-byte store per lane.
// Stores come from all eight compute waves, so no wave's store queue holds the workgroup back.
//
// Filter-stationary.  Each compute wave keeps its tile's filter in registers (KB x 4 fragments
// of 16 bytes per lane).  Row i of row block j holds channel 16*(i/4) + 4j + i%4, so lane
// (rho, g) ends with channels 16g .. 16g + 15 of pixel rho: one contiguous 16-byte output.
// The compute waves load the filter slice, bias and scales themselves (global -> LDS DMA,
// spread over the eight), wait for their own share and count it in an LDS word; each starts
// once the count reaches eight.
//
// Loader waves (waves 8 .. 11).  Loader l loads the range's input segments l, l + 4, ... in
// order (one 1 KB buffer_load ... lds per 8 pixels x 128 channel bytes or 16 pixels x 64,
// global -> LDS without registers).  It keeps a fixed number of segments in flight: after
// issuing its k-th segment it waits (vmcnt, a compile-time count) for its segment k - F and
// publishes the count of its landed segments in its own LDS word (lds_publish: a store that
// does not wait for the loader's later loads); a compute wave polls the word of the segment's
// loader (relaxed atomic loads, s_sleep between polls, bounded) before reading the segment.
// Loaders issue no stores, so their vmcnt waits count their own loads only, and the compute
// waves never wait on vmcnt after the filter.  LDS operations of one wave complete in order,
// so a count seen raised means the segments below it are in LDS.  Loader 0 zeroes the count
// words before the one barrier of the kernel.
//
// LDS layout (16-byte slots).  Input segment s of the range, pixel p (0..15) of it, chunk u
// (16 channels): slot s*16*C/16 + p*C/16 + (u ^ f(p)), f(p) = (p >> 1) & 7 (C = 128) or
// 2*((p >> 3) & 1) (C = 64).  Filter channel c (0 .. NT*64 - 1), chunk u: slot c*C/16 +
// (u ^ h(c)), h(c) = (2*(c >> 4) ^ (c & 3)) & 7 (C = 128) or 2*((c >> 4) & 1) (C = 64).
// The loads place each 16-byte chunk at its swizzled slot (a lane's source offset is the
// permuted one; every instruction still reads one contiguous kilobyte).  With these swizzles
// every ds_read_b128 of an MFMA fragment meets each LDS cycle's 16 lanes in 16 distinct slot
// classes (the half-wave, equal-popcount-parity lane-quad rule measured on gfx950).
//
// Epilogue.  Accumulators start at the bias (the first MFMA's C operand is the bias registers);
// the output is convert, scale, clamp, round (the 1.5*2^23 addition, bytes packed with
// v_perm_b32), the arithmetic of the other int8 kernels, interleaved with the next
// segment's matrix instructions (mma_requant_steps).  Every 16-byte store is followed by store_gap() on its data registers.

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kPwCompute = 8;                // compute waves
constexpr int kPwLoaders = 4;                // loader waves
constexpr int kPwThreads = 64 * (kPwCompute + kPwLoaders);
constexpr int kPwLds = 160 * 1024;
constexpr int kPwCount = 0;                  // LDS byte offset: [0] compute waves whose filter share landed,
                                             // [1 + l] loader l's segments landed
constexpr int kPwEp = 1024;                  // bias (1 KB, 256 entries max) then scales (1 KB)
constexpr int kPwFilt = 3072;                // the filter slice
constexpr int kPwInFlight = 22;              // loader: segments in flight (x KB instructions)
constexpr int kPwPerCu = 1;                  // workgroups per CU

__host__ __device__ constexpr int pw_filt_bytes(int NT, int KB) { return NT * 64 * KB * 64; }
__host__ __device__ constexpr int pw_input_lds(int NT, int KB) { return kPwFilt + pw_filt_bytes(NT, KB); }

struct PwArgs {
  const int8_t* x;
  const int8_t* w;
  const int32_t* bias;
  const float* wscale;
  int8_t* y;
  int P;        // pixels
  int K;        // output channels
  int nseg;     // ceil(P / 16)
  int nranges;  // segment ranges, a multiple of 8
  int ngroups;  // channel-tile groups (K / (64 * NT))
  float act_scale;
};

static_assert(sizeof(PwArgs) <= 256, "kernel arguments fit one s_load batch");

__device__ __forceinline__ unsigned pw_lds_addr(const void* p) {
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>(p) & 0xffffffffu);
}

// s_waitcnt vmcnt(N) for a compile-time 0 <= N <= 63.
template <int N>
__device__ __forceinline__ void pw_wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0xF70 | (N & 15) | ((N >> 4) << 14));
}

// swizzled chunk of input pixel p (of its segment) and of filter channel c
template <int KB>
__device__ __forceinline__ int pw_fin(int p) {
  return KB == 2 ? ((p >> 1) & 7) : 2 * ((p >> 3) & 1);
}
template <int KB>
__device__ __forceinline__ int pw_ffilt(int c) {
  return KB == 2 ? ((2 * (c >> 4)) ^ (c & 3)) & 7 : 2 * ((c >> 4) & 1);
}

// The loader's drain: after the last segment is issued, segments nseg - D .. nseg - 1 land one
// by one (D = min(nseg, F) of them in flight).  Step M waits for vmcnt <= M*KB (when M < D) and
// publishes nseg - M landed segments.
template <int KB, int M>
__device__ __forceinline__ void pw_drain(int D, int nseg, int* count, int lane) {
  if constexpr (M >= 0) {
    if (M < D) {
      pw_wait_vm<M * KB>();
      if (lane == 0) lds_publish(count, nseg - M);
    }
    pw_drain<KB, M - 1>(D, nseg, count, lane);
  }
}

template <int NT, int KB, bool RELU>
__global__ void __launch_bounds__(kPwThreads) i8_pointwise_kernel(PwArgs a_in) {
  constexpr int C = 64 * KB;              // input channels
  constexpr int kStreams = kPwCompute / NT;
  constexpr int kSegBytes = 16 * C;       // one input segment in LDS
  const PwArgs a = preload_args(a_in);
  extern __shared__ v4i smem[];
  const unsigned base = pw_lds_addr(smem);
  int* count = reinterpret_cast<int*>(reinterpret_cast<char*>(smem) + kPwCount);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // workgroup -> (range, channel group): the ngroups workgroups of a range share an XCD
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int i8 = bid >> 3;
  const int grp = i8 % a.ngroups;
  const int range = (i8 / a.ngroups) * 8 + xcd;
  const int s0 = static_cast<int>(static_cast<long long>(range) * a.nseg / a.nranges);
  const int s1 = static_cast<int>(static_cast<long long>(range + 1) * a.nseg / a.nranges);
  const int nseg = s1 - s0;
  const int k0 = grp * NT * 64;

  if (wave >= kPwCompute) {
    // ---- loader l: segments l, l + L, ... of the range (loader 0 first loads the filter) ----
    const int l = wave - kPwCompute;
    if (l == 0 && lane <= kPwLoaders)
      __hip_atomic_store(count + lane, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zeroed words are written
    barrier_only();
    // input: segment s is KB instructions of 16/KB pixels each; lane l of instruction j reads
    // pixel 16s + (16/KB)*j + l/(4KB), chunk (l % 4KB) ^ f(pixel); pixels past P read zeros
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.P * C);
    const int pl = lane / (4 * KB);                      // pixel of the instruction
    const int ul = lane - pl * 4 * KB;
    unsigned voff[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int p = (16 / KB) * j + pl;                  // pixel within the segment
      voff[j] = static_cast<unsigned>(p * C + 16 * (ul ^ pw_fin<KB>(p)));
    }
    const unsigned in_lds = static_cast<unsigned>(pw_input_lds(NT, KB)) / 16;
    // this loader's k-th segment: s = l + L*k
    auto issue = [&](int k) {
      const int s = l + kPwLoaders * k;
      const unsigned soff = static_cast<unsigned>(s0 + s) * kSegBytes;
#pragma unroll
      for (int j = 0; j < KB; ++j)
        load_lds16(rx, smem + in_lds + (kSegBytes / 16) * s + 64 * j, voff[j] + soff, 0);
    };
    const int nk = nseg > l ? (nseg - l + kPwLoaders - 1) / kPwLoaders : 0;
    int* mine = count + 1 + l;
    const int D = min(nk, kPwInFlight);
    for (int k = 0; k < D; ++k) issue(k);
    for (int k = D; k < nk; ++k) {
      issue(k);
      pw_wait_vm<kPwInFlight * KB>();  // this loader's segment k - F has landed
      if (lane == 0) lds_publish(mine, k - kPwInFlight + 1);
    }
    pw_drain<KB, kPwInFlight - 1>(D, nk, mine, lane);
    return;
  }

  barrier_only();  // the loader's zeroed words are visible

  // ---- the filter slice, bias and scales into LDS, spread over the compute waves (which
  // have no other loads or stores outstanding yet); each then counts its share landed ----
  {
    // instruction i fills slots 64i .. 64i + 63 = channel c, swizzled chunk u'
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + static_cast<size_t>(k0) * C, NT * 64 * C);
    for (int i = wave; i < NT * KB * 4; i += kPwCompute) {
      const int slot = 64 * i + lane;
      const int c = slot / (4 * KB);
      const int u = (slot - c * 4 * KB) ^ pw_ffilt<KB>(c);
      load_lds16(rw, smem + kPwFilt / 16 + 64 * i, static_cast<unsigned>(c * C + 16 * u), 0);
    }
    // bias and scales of the NT*64 channels (past them: zeros)
    if (wave == kPwCompute - 2) {
      load_lds16(make_rsrc(a.bias ? a.bias + k0 : nullptr, a.bias ? NT * 256 : 0), smem + kPwEp / 16, 16u * lane, 0);
    } else if (wave == kPwCompute - 1) {
      load_lds16(make_rsrc(a.wscale + k0, NT * 256), smem + (kPwEp + 1024) / 16, 16u * lane, 0);
    }
  }
  wait_vmcnt(0);
  if (lane == 0) __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  const int t = wave % NT;
  const int st = wave / NT;
  const int rho = lane & 15;
  const int g = lane >> 4;
  auto poll = [&](int word, int need) {
    // bounded: the loader publishes every count, so this ends long before the bound
    for (int it = 0; it < (1 << 22); ++it) {
      if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(count + word, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_WORKGROUP)) >= need)
        break;
      __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
  };
  poll(0, kPwCompute);  // every compute wave's share of the filter has landed

  // filter fragments: A[b][j], lane (rho, g) = channel 64t + 16*(rho/4) + 4j + rho%4, chunk 4b + g
  v4i A[KB][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = 64 * t + 16 * (rho >> 2) + 4 * j + (rho & 3);
#pragma unroll
    for (int b = 0; b < KB; ++b)
      A[b][j] = lds_read16(base + kPwFilt + 16u * static_cast<unsigned>(4 * KB * c + ((4 * b + g) ^ pw_ffilt<KB>(c))));
  }
  // bias and requantization multipliers of the lane's channels 64t + 16g + 4j + i
  v4i bias_v[4];
  v4f mult_v[4];
  const unsigned bias_a = base + kPwEp + 4u * static_cast<unsigned>(64 * t + 16 * g);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bias_v[j] = lds_read16(bias_a + 16u * j);
    const v4i ws = lds_read16(bias_a + 16u * j + 1024u);
#pragma unroll
    for (int i = 0; i < 4; ++i) mult_v[j][i] = requant_multiplier(a.act_scale, __int_as_float(ws[i]));
  }

  // this lane's B fragment of K-block b in segment s: pixel rho, chunk 4b + g
  unsigned boff[KB];
#pragma unroll
  for (int b = 0; b < KB; ++b)
    boff[b] = base + static_cast<unsigned>(pw_input_lds(NT, KB)) +
              16u * static_cast<unsigned>(4 * KB * rho + ((4 * b + g) ^ pw_fin<KB>(rho)));
  // output: pixel 16s + rho of the range, channels k0 + 64t + 16g ..; pixels past P dropped
  const size_t out0 = static_cast<size_t>(s0) * 16 * a.K + k0 + 64 * t;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y + out0, (a.P - 16 * s0) * a.K - k0 - 64 * t);
  const unsigned ylane = static_cast<unsigned>(rho * a.K + 16 * g);

  // segment s comes from loader s % L as its (s / L)-th; a stream's segments all come from
  // one loader (the stream count is a multiple of L)
  static_assert(kStreams % kPwLoaders == 0, "streams map to one loader each");
  const int word = 1 + st % kPwLoaders;
  int seen = 0;
  auto wait_seg = [&](int s) {
    const int need = s / kPwLoaders + 1;
    if (seen < need) {
      poll(word, need);
      seen = __builtin_amdgcn_readfirstlane(
          __hip_atomic_load(count + word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    }
  };
  // the MFMAs of segment s into acc (started at the bias)
  auto mma = [&](int s, v4i (&acc)[4]) {
    v4i B[KB];
#pragma unroll
    for (int b = 0; b < KB; ++b) B[b] = lds_read16(boff[b] + static_cast<unsigned>(s) * kSegBytes);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0][j], B[0], bias_v[j], 0, 0, 0);
#pragma unroll
    for (int b = 1; b < KB; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b], acc[j], 0, 0, 0);
  };
  // the store offset of this wave's current segment; pixels past P lie past num_records
  // ((P - 16 s0) * K - k0 - 64t bytes from the tile's first byte) and are dropped
  unsigned yoff = static_cast<unsigned>(st) * 16u * static_cast<unsigned>(a.K) + ylane;
  const unsigned ystep = static_cast<unsigned>(kStreams) * 16u * static_cast<unsigned>(a.K);
  auto emit = [&](const v4i (&acc)[4]) {
    const v4i pk = RELU ? pack_u8_relu(acc, mult_v) : pack_i8(acc, mult_v, -128.0f);
    __builtin_amdgcn_raw_buffer_store_b128(pk, ry, yoff, 0, kStoreAux);
    store_gap(pk);
    yoff += ystep;
  };
  // Software-pipelined by one segment: each matrix instruction of the next segment is issued
  // with a share of this segment's output stage (mma_requant_steps), so the two overlap.
  int s = st;
  if (s < nseg) {
    v4i acc[4];
    wait_seg(s);
    mma(s, acc);
    for (;;) {
      const int sn = s + kStreams;
      if (sn >= nseg) break;
      wait_seg(sn);
      v4i B[KB];
#pragma unroll
      for (int b = 0; b < KB; ++b) B[b] = lds_read16(boff[b] + static_cast<unsigned>(sn) * kSegBytes);
      v4i accn[4];
      unsigned pk[4];
      float f[16];
      mma_requant_steps<KB>(A, B, bias_v, accn, acc, mult_v, RELU ? 0.0f : -128.0f, f, pk);
      const v4i pkv = {static_cast<int>(pk[0]), static_cast<int>(pk[1]), static_cast<int>(pk[2]),
                       static_cast<int>(pk[3])};
      __builtin_amdgcn_raw_buffer_store_b128(pkv, ry, yoff, 0, kStoreAux);
      store_gap(pkv);
      yoff += ystep;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = accn[j];
      s = sn;
    }
    emit(acc);
  }
}

struct PwPlan {
  int NT, KB, nseg, nranges, ngroups, segs_max;
  size_t lds;
};

bool pw_plan(const Geom& g, PwPlan* p, std::string* why) {
  auto no = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (g.G != 1) return no("pointwise kernel needs groups == 1");
  if (g.R != 1 || g.S != 1) return no("pointwise kernel needs a 1x1 filter");
  if (g.sh != 1 || g.sw != 1 || g.ph != 0 || g.pw != 0) return no("pointwise kernel needs stride 1 and no padding");
  if (g.C != 64 && g.C != 128) return no("pointwise kernel needs 64 or 128 input channels");
  if (g.K % 64 != 0 || g.K <= 0) return no("pointwise kernel needs k % 64 == 0");
  const long long P = static_cast<long long>(g.N) * g.Ho * g.Wo;
  if (P <= 0) return no("pointwise kernel needs a non-empty output");
  if (P * g.C >= (1LL << 31) || P * g.K >= (1LL << 30)) return no("pointwise kernel needs tensors below 2^30 bytes");
  p->KB = g.C / 64;
  p->NT = g.K % 128 == 0 ? 2 : 1;
  p->ngroups = g.K / (64 * p->NT);
  p->nseg = static_cast<int>((P + 15) / 16);
  const int seg_bytes = 16 * g.C;
  p->segs_max = (kPwLds / kPwPerCu - pw_input_lds(p->NT, p->KB)) / seg_bytes;
  // kPwPerCu workgroups per CU: ranges x groups ~ that many per CU, more where a range would
  // not fit
  const int slots = 256 * kPwPerCu;
  long long nr = std::max<long long>((slots + p->ngroups - 1) / p->ngroups, (p->nseg + p->segs_max - 1) / p->segs_max);
  nr = (nr + 7) / 8 * 8;
  if (nr * p->ngroups > 0x7fffffffLL) return no("grid too large");
  p->nranges = static_cast<int>(nr);
  const int per = (p->nseg + p->nranges - 1) / p->nranges;
  p->lds = static_cast<size_t>(pw_input_lds(p->NT, p->KB)) + static_cast<size_t>(per) * seg_bytes;
  if (p->lds > static_cast<size_t>(kPwLds / kPwPerCu)) return no("pointwise kernel range does not fit in LDS");
  return true;
}

bool pw_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool pointwise_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                        std::string* why) {
  if (epi != kEpiI8) {
    if (why) *why = "pointwise kernel: int8 outputs only";
    return false;
  }
  if (!pw_aligned16(x) || !pw_aligned16(w) || !pw_aligned16(y) || !pw_aligned16(rq.wscale) ||
      (rq.bias && !pw_aligned16(rq.bias))) {
    if (why) *why = "pointwise kernel needs 16-byte aligned x, w, y, bias and scales";
    return false;
  }
  PwPlan pl;
  return pw_plan(g, &pl, why);
}

hipError_t launch_i8_pointwise(const Geom& g, const int8_t* x, const int8_t* w, int8_t* y, const Requant& rq,
                               hipStream_t stream) {
  PwPlan pl;
  if (!pw_plan(g, &pl, nullptr)) return hipErrorInvalidConfiguration;
  PwArgs a;
  a.x = x;
  a.w = w;
  a.bias = rq.bias;
  a.wscale = rq.wscale;
  a.y = y;
  a.P = g.N * g.Ho * g.Wo;
  a.K = g.K;
  a.nseg = pl.nseg;
  a.nranges = pl.nranges;
  a.ngroups = pl.ngroups;
  a.act_scale = rq.act_scale;
  const unsigned blocks = static_cast<unsigned>(pl.nranges) * static_cast<unsigned>(pl.ngroups);
  auto go = [&](auto kern) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(pl.lds));
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kPwThreads), pl.lds, stream, a);
  };
  const bool relu = rq.relu != 0;
  if (pl.NT == 2) {
    if (pl.KB == 2) relu ? go(i8_pointwise_kernel<2, 2, true>) : go(i8_pointwise_kernel<2, 2, false>);
    else relu ? go(i8_pointwise_kernel<2, 1, true>) : go(i8_pointwise_kernel<2, 1, false>);
  } else {
    if (pl.KB == 2) relu ? go(i8_pointwise_kernel<1, 2, true>) : go(i8_pointwise_kernel<1, 2, false>);
    else relu ? go(i8_pointwise_kernel<1, 1, true>) : go(i8_pointwise_kernel<1, 1, false>);
  }
  return hipGetLastError();
}

}  // namespace miq
