// int32 batched GEMM on the int8 matrix cores: C[b] = op(A[b]) * op(B[b]) with int32
// wrap-around arithmetic, the semantics of the reference's bmm_matmul_i32
// (/root/reference/bmm.cu:155-246, :298-322), exact for every int32 input.
//
// Digits.  Every int32 u is, modulo 2^32, d0 + 256 d1 + 2^16 d2 + 2^24 d3 with signed
// digits d_i in [-128, 127]; the bytes of w = (u + 0x808080) ^ 0x808080 are exactly those
// digits (adding 128 to the low three bytes and subtracting it again per byte carries the
// balanced representation).  A product a * b is then, modulo 2^32,
//   S0 + 2^8 S1 + 2^16 S2 + 2^24 S3,   S_s = sum over i + j = s of d_i(a) e_j(b),
// the terms with i + j >= 4 vanishing.  v_mfma_i32_16x16x64_i8 multiplies 64 byte pairs
// and sums them: fed A's digit words as they are and B's digit words byte-reversed and
// shifted right by 8 * (3 - s), byte p of A meets e_{s-p} of B (zero where s - p < 0), so
// one MFMA K-block of 16 k values gives S_s for those k.  Four accumulator sets (s = 0..3)
// and a final shift-and-add give the exact wrapped product sums; each S_s may itself wrap,
// as only S_s mod 2^(32 - 8s) matters.
//
// Work decomposition.  A workgroup of 8 waves computes 128 (m) x 64 (n) of one batch
// entry; wave w computes n 32 * (w % 2) .. +31 and m 32 * (w / 2) .. +31: 2 x 2 MFMA tiles
// x 4 shift groups.  The MFMA's A operand is B's rows (n) and its B operand A's rows (m),
// so a lane's accumulators hold 4 consecutive n of one m: one 16-byte store of C.
//
// Staging.  Chunks of 16 k values are loaded to registers (zero outside the matrices:
// zero's digits are zero), turned into digit words (byte-reversed for B) and stored to a
// double-buffered LDS tile, [row][k] with 64-byte rows whose 16-byte chunk g sits at
// g ^ (2 * bit 3 of the row): a fragment read (16 rows, one chunk per lane group) is then
// free of bank conflicts under the ds_read_b128 rule (16 lanes per cycle: one half-wave's
// lane quads of equal quad-index parity, distinct 16-byte slots modulo 16).

#include "qconv_device.h"

#include <algorithm>

namespace miq {
namespace {

constexpr int kGemmWaves = 8;
constexpr int kGemmBM = 128;  // m per workgroup
constexpr int kGemmBN = 64;   // n per workgroup
constexpr int kGemmKC = 16;   // k values per chunk: one MFMA K-block of digit bytes
constexpr int kGemmDepth = 2; // chunks in flight per thread (2: <= 116 VGPRs, two workgroups per CU; measured faster than 3 or 4)

typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

struct GemmArgs {
  const int32_t* A;
  const int32_t* B;
  int32_t* C;
  int M, N, K;
  int tn;        // n tiles
  int tiles;     // m tiles * n tiles per batch entry
  int nchunks;   // ceil(K / 16)
  int b0;        // first batch entry of this launch
  FastDivM fd_tn, fd_tiles;
};

__device__ __forceinline__ unsigned digit_word(unsigned u) { return (u + 0x808080u) ^ 0x808080u; }

// 16-byte slot of (row, chunk g) in a staged tile
__device__ __forceinline__ int tile_slot(int row, int g) { return 4 * row + (g ^ (((row >> 3) & 1) << 1)); }

// Loads of one thread for chunk c, on one straight code path for every chunk: the k
// index is clamped to the row (k <= K - 1, or the last 4 / 2 values for a vector read), so
// every load stays inside its matrix and none is skipped; values of k >= K (only the last
// chunk has them) are zeroed when the chunk is staged.  Rows past M (N) are read from the
// last row: they only feed output rows (columns) that are never stored.  With the same
// loads on every path the compiler's counters of the loads in flight stay exact across the
// pipelined loop.  VA / VB: K-contiguous rows read as one 16- (8-) byte load (K % 4 == 0
// and a 16-byte aligned A; K % 2 == 0 and an 8-byte aligned B).
template <bool TA, bool TB, bool VA, bool VB>
struct GemmLoader {
  const int32_t* ra;  // A value (this thread's row or column, k = 0)
  const int32_t* rb;
  size_t sa, sb;      // element distance between consecutive k
  int ka, kb;         // this thread's first k within a chunk (A, B)
  int K;

  __device__ __forceinline__ void load(int c, unsigned (&v)[4], unsigned (&w)[2]) const {
    const int k0 = c * kGemmKC;
    if constexpr (VA) {
      const v4i t = *reinterpret_cast<const v4i*>(ra + min(k0 + ka, K - 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = static_cast<unsigned>(t[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = static_cast<unsigned>(ra[static_cast<size_t>(min(k0 + ka + e, K - 1)) * sa]);
    }
    if constexpr (VB) {
      const v2i t = *reinterpret_cast<const v2i*>(rb + min(k0 + kb, K - 2));
      w[0] = static_cast<unsigned>(t[0]);
      w[1] = static_cast<unsigned>(t[1]);
    } else {
#pragma unroll
      for (int e = 0; e < 2; ++e) w[e] = static_cast<unsigned>(rb[static_cast<size_t>(min(k0 + kb + e, K - 1)) * sb]);
    }
  }

  // zeroes the values of k >= K of chunk c (a no-op except on the last chunk)
  __device__ __forceinline__ void mask(int c, unsigned (&v)[4], unsigned (&w)[2]) const {
    const int k0 = c * kGemmKC;
    if (k0 + kGemmKC > K) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = k0 + ka + e < K ? v[e] : 0u;
#pragma unroll
      for (int e = 0; e < 2; ++e) w[e] = k0 + kb + e < K ? w[e] : 0u;
    }
  }
};

// This wave's LDS writes complete, then the workgroup barrier; pending global loads stay
// in flight (no vmcnt wait), and the clobber keeps LDS accesses on their side of it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(64 * kGemmWaves, 1) i32_gemm_kernel(GemmArgs a) {
  __shared__ v4i sA[2][kGemmBM * 4];
  __shared__ v4i sB[2][kGemmBN * 4];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);

  const int lin = blockIdx.x;
  const int bl = fdiv(lin, a.fd_tiles);
  const int rem = lin - bl * a.tiles;
  const int bi = a.b0 + bl;
  const int tmi = fdiv(rem, a.fd_tn);
  const int tni = rem - tmi * a.tn;
  const int m0 = tmi * kGemmBM;
  const int n0 = tni * kGemmBN;
  const int32_t* Ab = a.A + static_cast<size_t>(bi) * a.M * a.K;
  const int32_t* Bb = a.B + static_cast<size_t>(bi) * a.K * a.N;
  int32_t* Cb = a.C + static_cast<size_t>(bi) * a.M * a.N;

  // staging assignment: A 128 rows x 16 k, 4 k values per thread; B 64 rows x 16 k, 2 per
  // thread.  K-contiguous operands: a thread's values are adjacent in memory; M- or
  // N-contiguous ones: adjacent lanes take adjacent rows.
  const int ar = TA ? (t & 127) : (t >> 2);
  const int aq = TA ? (t >> 7) : (t & 3);
  const int br = TB ? (t >> 3) : (t & 63);
  const int bp = TB ? (t & 7) : (t >> 6);
  const int am = min(m0 + ar, a.M - 1);
  const int bn = min(n0 + br, a.N - 1);
  GemmLoader<TA, TB, VA, VB> ld;
  ld.ra = TA ? Ab + am : Ab + static_cast<size_t>(am) * a.K;
  ld.rb = TB ? Bb + static_cast<size_t>(bn) * a.K : Bb + bn;
  ld.sa = TA ? static_cast<size_t>(a.M) : 1;
  ld.sb = TB ? 1 : static_cast<size_t>(a.N);
  ld.ka = 4 * aq;
  ld.kb = 2 * bp;
  ld.K = a.K;

  const int sa_slot = tile_slot(ar, aq);
  const int sb_slot = tile_slot(br, bp >> 1);
  auto stage = [&](int buf, int c, unsigned (&va)[4], unsigned (&vb)[2]) {
    ld.mask(c, va, vb);
    sA[buf][sa_slot] = v4i{static_cast<int>(digit_word(va[0])), static_cast<int>(digit_word(va[1])),
                           static_cast<int>(digit_word(va[2])), static_cast<int>(digit_word(va[3]))};
    v2i* pb = reinterpret_cast<v2i*>(&sB[buf][sb_slot]) + (bp & 1);
    *pb = v2i{static_cast<int>(__builtin_bswap32(digit_word(vb[0]))),
              static_cast<int>(__builtin_bswap32(digit_word(vb[1])))};
  };

  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int fb0 = tile_slot(32 * wn + (lane & 15), lane >> 4);
  const int fb1 = tile_slot(32 * wn + 16 + (lane & 15), lane >> 4);
  const int fa0 = tile_slot(32 * wm + (lane & 15), lane >> 4);
  const int fa1 = tile_slot(32 * wm + 16 + (lane & 15), lane >> 4);
  v4i acc[4][2][2];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int jn = 0; jn < 2; ++jn)
#pragma unroll
      for (int im = 0; im < 2; ++im) acc[s][jn][im] = v4i{0, 0, 0, 0};

  // kGemmDepth chunks in flight in registers: set j % depth holds chunk j from its load
  // until it is staged to LDS, one chunk before its MFMAs
  constexpr int P = kGemmDepth;
  const int nch = a.nchunks;
  unsigned va[P][4], vb[P][2];
  // The loop runs whole groups of kGemmDepth chunks; chunks past the last are loaded as the
  // last one again and staged as zeros (their k are all >= K), so their MFMAs add nothing.
  // Every pass thus loads, computes and stages on one code path, and the counters of the
  // loads in flight are the same on every path.  K == 0 loads nothing (the operands may be
  // empty) and stores zeros.
  if (nch > 0) {
    const int last = nch - 1;
#pragma unroll
    for (int j = 0; j < P; ++j) ld.load(min(j, last), va[j], vb[j]);
    stage(0, 0, va[0], vb[0]);
    lds_barrier();
    for (int c0 = 0; c0 < nch; c0 += P) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int c = c0 + j;
        ld.load(min(c + P, last), va[j], vb[j]);  // set j was staged last iteration
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
        stage(buf ^ 1, c + 1, va[(j + 1) % P], vb[(j + 1) % P]);
        lds_barrier();
      }
    }
  }

  // lane (c = lane % 16, g = lane / 16) of tile (jn, im): m = 32 wm + 16 im + c,
  // n = 32 wn + 16 jn + 4 g .. + 3
  const bool vec = (a.N & 3) == 0 && (reinterpret_cast<uintptr_t>(a.C) & 15u) == 0;
#pragma unroll
  for (int jn = 0; jn < 2; ++jn) {
#pragma unroll
    for (int im = 0; im < 2; ++im) {
      const int m = m0 + 32 * wm + 16 * im + (lane & 15);
      const int nb = n0 + 32 * wn + 16 * jn + 4 * (lane >> 4);
      v4i r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned v = static_cast<unsigned>(acc[0][jn][im][i]) + (static_cast<unsigned>(acc[1][jn][im][i]) << 8) +
                           (static_cast<unsigned>(acc[2][jn][im][i]) << 16) +
                           (static_cast<unsigned>(acc[3][jn][im][i]) << 24);
        r[i] = static_cast<int>(v);
      }
      if (m >= a.M) continue;
      int32_t* crow = Cb + static_cast<size_t>(m) * a.N;
      if (vec && nb + 3 < a.N) {
        *reinterpret_cast<v4i*>(crow + nb) = r;
        store_gap(r);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (nb + i < a.N) crow[nb + i] = r[i];
      }
    }
  }
}

template <bool TA, bool TB, bool VA, bool VB>
void gemm_launch(const GemmArgs& a, unsigned blocks, hipStream_t stream) {
  hipLaunchKernelGGL((i32_gemm_kernel<TA, TB, VA, VB>), dim3(blocks), dim3(64 * kGemmWaves), 0, stream, a);
}

}  // namespace

hipError_t launch_i32_gemm(const int32_t* A, const int32_t* B, int32_t* C, int batch, int M, int N, int K, bool ta,
                           bool tb, hipStream_t stream) {
  if (batch == 0 || M == 0 || N == 0) return hipSuccess;
  GemmArgs a;
  a.A = A; a.B = B; a.C = C;
  a.M = M; a.N = N; a.K = K;
  a.tn = (N + kGemmBN - 1) / kGemmBN;
  const int tm = (M + kGemmBM - 1) / kGemmBM;
  const long long tiles = static_cast<long long>(tm) * a.tn;
  // a launch stays below 2^31 work-items: at most kMaxBlocks workgroups of 512
  constexpr long long kMaxBlocks = 1LL << 22;
  if (tiles > kMaxBlocks) return hipErrorInvalidConfiguration;
  a.tiles = static_cast<int>(tiles);
  a.nchunks = (K + kGemmKC - 1) / kGemmKC;
  a.fd_tn = fastdiv_m(a.tn);
  a.fd_tiles = fastdiv_m(a.tiles);
  const bool va = !ta && (K & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
  const bool vb = tb && (K & 1) == 0 && (reinterpret_cast<uintptr_t>(B) & 7u) == 0;
  const long long per_launch = std::min<long long>(batch, kMaxBlocks / tiles);
  for (long long b0 = 0; b0 < batch; b0 += per_launch) {
    a.b0 = static_cast<int>(b0);
    const unsigned nb = static_cast<unsigned>(std::min<long long>(per_launch, batch - b0) * tiles);
    if (!ta && !tb) {
      if (va) gemm_launch<false, false, true, false>(a, nb, stream);
      else gemm_launch<false, false, false, false>(a, nb, stream);
    } else if (!ta && tb) {
      if (va && vb) gemm_launch<false, true, true, true>(a, nb, stream);
      else if (va) gemm_launch<false, true, true, false>(a, nb, stream);
      else if (vb) gemm_launch<false, true, false, true>(a, nb, stream);
      else gemm_launch<false, true, false, false>(a, nb, stream);
    } else if (ta && !tb) {
      gemm_launch<true, false, false, false>(a, nb, stream);
    } else {
      if (vb) gemm_launch<true, true, false, true>(a, nb, stream);
      else gemm_launch<true, true, false, false>(a, nb, stream);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace miq
