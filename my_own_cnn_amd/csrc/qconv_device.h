// Device helpers shared by the MFMA convolution kernels: operand types, unaligned LDS
// reads and the fused output stage for one lane's 16 consecutive output channels.
#pragma once

#include "qconv_internal.h"

namespace miq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Cache policy of the int8 kernels' output stores: non-temporal (nt) with system-scope
// write-through (sc0 | sc1), so the next kernel does not have to write this one's output
// back from L2 before its own loads.  Measured against nt alone: 3-5% per launch on the
// row-band kernels (r50_3x3 7.05 -> 6.8 us); plain write-back stores are 10-20% slower.
constexpr int kStoreAux = 19;  // sc0 (1) | nt (2) | sc1 (16)

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// FastDiv without its divisor (the device only needs the multiplier and the shift).
struct FastDivM {
  uint32_t m, s;
};
inline FastDivM fastdiv_m(uint32_t d) {
  const FastDiv f = make_fastdiv(d);
  return FastDivM{f.m, f.s};
}
__device__ __forceinline__ int fdiv(int n, const FastDivM& f) {
  const uint32_t un = static_cast<uint32_t>(n);
  return static_cast<int>((__umulhi(un, f.m) + un) >> f.s);
}

// Workgroup id -> tile index such that each of the 8 XCDs (workgroups are dealt to them
// round-robin) gets one contiguous range of tiles: neighbouring tiles share an L2.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
  const int q = total >> 3;
  const int r = total & 7;
  const int xcd = bid & 7;
  const int pos = bid >> 3;
  return xcd * q + min(xcd, r) + pos;
}

// s_waitcnt vmcnt(n) for a wave-uniform 0 <= n <= 63 (the counter's full 6 bits: bits 3:0 and
// 15:14 of the immediate); counts above 63 wait for 63, which is always correct.
__device__ __forceinline__ void wait_vmcnt63(int n) {
#define MIQ_VMCNT_CASE(k) \
  case k: __builtin_amdgcn_s_waitcnt(0xF70 | ((k) & 15) | (((k) >> 4) << 14)); break;
#define MIQ_VMCNT_CASE8(k) MIQ_VMCNT_CASE(k) MIQ_VMCNT_CASE(k + 1) MIQ_VMCNT_CASE(k + 2) MIQ_VMCNT_CASE(k + 3) \
  MIQ_VMCNT_CASE(k + 4) MIQ_VMCNT_CASE(k + 5) MIQ_VMCNT_CASE(k + 6) MIQ_VMCNT_CASE(k + 7)
  switch (n <= 0 ? 0 : (n >= 63 ? 63 : n)) {
    MIQ_VMCNT_CASE8(0) MIQ_VMCNT_CASE8(8) MIQ_VMCNT_CASE8(16) MIQ_VMCNT_CASE8(24)
    MIQ_VMCNT_CASE8(32) MIQ_VMCNT_CASE8(40) MIQ_VMCNT_CASE8(48) MIQ_VMCNT_CASE8(56)
    default: break;
  }
#undef MIQ_VMCNT_CASE8
#undef MIQ_VMCNT_CASE
}

// s_waitcnt vmcnt(n) for a wave-uniform n; counts above 15 wait for 15 (waiting for more
// completions than needed is always correct).
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n <= 0 ? 0 : (n >= 15 ? 15 : n)) {
    case 0: __builtin_amdgcn_s_waitcnt(0xF70 | 0); break;
    case 1: __builtin_amdgcn_s_waitcnt(0xF70 | 1); break;
    case 2: __builtin_amdgcn_s_waitcnt(0xF70 | 2); break;
    case 3: __builtin_amdgcn_s_waitcnt(0xF70 | 3); break;
    case 4: __builtin_amdgcn_s_waitcnt(0xF70 | 4); break;
    case 5: __builtin_amdgcn_s_waitcnt(0xF70 | 5); break;
    case 6: __builtin_amdgcn_s_waitcnt(0xF70 | 6); break;
    case 7: __builtin_amdgcn_s_waitcnt(0xF70 | 7); break;
    case 8: __builtin_amdgcn_s_waitcnt(0xF70 | 8); break;
    case 9: __builtin_amdgcn_s_waitcnt(0xF70 | 9); break;
    case 10: __builtin_amdgcn_s_waitcnt(0xF70 | 10); break;
    case 11: __builtin_amdgcn_s_waitcnt(0xF70 | 11); break;
    case 12: __builtin_amdgcn_s_waitcnt(0xF70 | 12); break;
    case 13: __builtin_amdgcn_s_waitcnt(0xF70 | 13); break;
    case 14: __builtin_amdgcn_s_waitcnt(0xF70 | 14); break;
    default: __builtin_amdgcn_s_waitcnt(0xF70 | 15); break;
  }
}

// Workgroup barrier without the memory fence of __syncthreads (which would wait for this
// wave's pending stores); the clobber keeps LDS accesses on their side of it.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), num_records, 0x00020000);
}

// 16 bytes per lane, global -> LDS at lds + 16 * lane; out-of-range lanes write zeros.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, v4i* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
}

// Writes v to the LDS word at p (a pointer into __shared__ memory) without waiting for this
// wave's outstanding loads.  After a buffer_load ... lds the compiler puts a vmcnt(0) wait in
// front of any LDS store, plain or atomic, because it cannot tell the loads' LDS destinations
// from the stored word apart: a loader wave that publishes its progress word by word would
// wait for all of its loads at the first publish.  The store is issued by inline assembly,
// which that analysis does not see; this wave's LDS operations still complete in order, and
// an LDS operation the compiler does not count only makes its lgkmcnt waits stricter.
__device__ __forceinline__ void lds_publish(int* p, int v) {
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p) & 0xffffffffu);
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}

// 16 bytes from LDS byte address `addr`.
__device__ __forceinline__ v4i lds_read16(unsigned addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(static_cast<uintptr_t>(addr));
}

// Four rounded values (each v + 1.5 * 2^23, so that its low byte is rint(v) in two's
// complement for |v| <= 128) packed into one word, low bytes in order: two v_perm_b32 and an
// or.
__device__ __forceinline__ unsigned pack4_magic(float a, float b, float c, float d) {
  return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0400u) |
         __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x04000c0cu);
}

// The int8 output stage of one value: clamp(rint(float(acc) * m), lo, 127) (lo = -128, or 0
// with ReLU), computed as med3(v, lo, 127) + 1.5 * 2^23: the bounds are integers, so clamping
// first equals rounding first, and the addition rounds to nearest even and leaves rint in the
// low byte.  v_med3_f32 returns its lower bound for a NaN input (the NaN rule of the
// reference's saturation).  Every step writes a fresh register: read-modify-write packing of
// one register (SDWA byte writes, v_cvt_pk_u8_f32 into a partly filled word) was measured to
// stall the wave behind the matrix instructions in flight, and took the overlap of MFMA and
// VALU work away.
__device__ __forceinline__ float requant_magic(int acc, float m, float lo) {
  return __builtin_amdgcn_fmed3f(static_cast<float>(acc) * m, lo, 127.0f) + 12582912.0f;
}

// int8 output of one lane: channels kc0 .. kc0 + 15 of one pixel (accumulator word j, value r
// = channel 4j + r), accumulators biased.
__device__ __forceinline__ v4i pack_i8(const v4i (&acc)[4], const v4f (&mult)[4], float lo) {
  v4i pk;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float c[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) c[r] = requant_magic(acc[j][r], mult[j][r], lo);
    pk[j] = static_cast<int>(pack4_magic(c[0], c[1], c[2], c[3]));
  }
  return pk;
}

// Values V .. VE - 1 (V = 4j + r) of a lane's 16 through requant_magic into f; each completed
// word (r == 3) is packed into pk[j].
template <int V, int VE>
__device__ __forceinline__ void requant_values(const v4i (&acc)[4], const v4f (&mult)[4], float lo, float (&f)[16],
                                               unsigned (&pk)[4]) {
  if constexpr (V < VE) {
    f[V] = requant_magic(acc[V / 4][V % 4], mult[V / 4][V % 4], lo);
    if constexpr (V % 4 == 3) pk[V / 4] = pack4_magic(f[V - 3], f[V - 2], f[V - 1], f[V]);
    requant_values<V + 1, VE>(acc, mult, lo, f, pk);
  }
}

// One software-pipelined segment step of the filter-stationary int8 kernels: the KB x 4
// MFMAs of the next segment (K-block I / 4, row block I % 4; the first K-block starts from the
// bias) each followed by its share of the current segment's 16 output values, with a
// scheduling barrier after each pair, so that each wave's output stage issues while its own
// matrix instructions execute.  (Left to itself the compiler puts all matrix instructions
// first and the output stage after them.)
template <int KB, int I = 0>
__device__ __forceinline__ void mma_requant_steps(const v4i (&A)[KB][4], const v4i (&B)[KB], const v4i (&bias)[4],
                                                  v4i (&accn)[4], const v4i (&acc)[4], const v4f (&mult)[4], float lo,
                                                  float (&f)[16], unsigned (&pk)[4]) {
  if constexpr (I < 4 * KB) {
    constexpr int b = I / 4;
    constexpr int j = I % 4;
    accn[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b], b == 0 ? bias[j] : accn[j], 0, 0, 0);
    requant_values<I * 16 / (4 * KB), (I + 1) * 16 / (4 * KB)>(acc, mult, lo, f, pk);
    __builtin_amdgcn_sched_barrier(0);
    mma_requant_steps<KB, I + 1>(A, B, bias, accn, acc, mult, lo, f, pk);
  }
}

// Stage S of value V (= 4j + r) of requant_magic, one instruction each: 0 convert, 1 scale,
// 2 clamp, 3 round (+ 1.5 * 2^23).  Same operations and order as requant_magic, so the same
// bits.
template <int V, int S>
__device__ __forceinline__ void requant_stage(const v4i (&acc)[4], const v4f (&mult)[4], float lo, float (&c)[16]) {
  if constexpr (V >= 0 && V < 16) {
    if constexpr (S == 0) c[V] = static_cast<float>(acc[V / 4][V % 4]);
    if constexpr (S == 1) c[V] = c[V] * mult[V / 4][V % 4];
    if constexpr (S == 2) c[V] = __builtin_amdgcn_fmed3f(c[V], lo, 127.0f);
    if constexpr (S == 3) c[V] = c[V] + 12582912.0f;
  }
}

// The output stage of gap I of a 16-MFMA segment step, software-pipelined over the values:
// stage 3 of value I - 3, 2 of I - 2, 1 of I - 1 and 0 of I, so the gap's four instructions
// are independent of each other (a value's four stages are a chain of dependent
// instructions, and one value per gap would issue them back to back).  A word is packed in
// the gap that rounds its last value.
template <int I>
__device__ __forceinline__ void requant_gap(const v4i (&acc)[4], const v4f (&mult)[4], float lo, float (&c)[16],
                                            unsigned (&pk)[4]) {
  requant_stage<I - 3, 3>(acc, mult, lo, c);
  requant_stage<I - 2, 2>(acc, mult, lo, c);
  requant_stage<I - 1, 1>(acc, mult, lo, c);
  requant_stage<I, 0>(acc, mult, lo, c);
  if constexpr (I - 3 >= 0 && I - 3 < 16 && (I - 3) % 4 == 3) {
    constexpr int V = I - 3;
    pk[V / 4] = pack4_magic(c[V - 3], c[V - 2], c[V - 1], c[V]);
  }
}

// mma_requant_steps for KB = 4 (one value per matrix instruction) with the pipelined output
// stage; the last three values' remaining stages (gaps 16 to 18) follow the last MFMA.
template <int I = 0>
__device__ __forceinline__ void mma_requant_pipe4(const v4i (&A)[4][4], const v4i (&B)[4], const v4i (&bias)[4],
                                                  v4i (&accn)[4], const v4i (&acc)[4], const v4f (&mult)[4], float lo,
                                                  float (&c)[16], unsigned (&pk)[4]) {
  if constexpr (I < 16) {
    constexpr int b = I / 4;
    constexpr int j = I % 4;
    accn[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b][j], B[b], b == 0 ? bias[j] : accn[j], 0, 0, 0);
    requant_gap<I>(acc, mult, lo, c, pk);
    __builtin_amdgcn_sched_barrier(0);
    mma_requant_pipe4<I + 1>(A, B, bias, accn, acc, mult, lo, c, pk);
  } else {
    requant_gap<16>(acc, mult, lo, c, pk);
    requant_gap<17>(acc, mult, lo, c, pk);
    requant_gap<18>(acc, mult, lo, c, pk);
  }
}

// Wait states after a 16-byte store before another instruction may overwrite its data
// registers.  A vector-memory store of more than 64 bits needs one wait state before a
// VALU write of its data VGPRs; the compiler leaves none when the store ends a loop body
// and the loop header's first instruction overwrites them (seen: buffer_store_dwordx4
// v[160:163] directly followed by v_add_u32 v160, and the first dword of some lanes
// stored wrong, varying from run to run).  Two wait states after every such store close
// that window: the statement reads the stored registers, so nothing may overwrite them
// before it, and its "memory" clobber keeps the store ahead of it.
template <typename V>
__device__ __forceinline__ void store_gap(const V& data) {
  asm volatile("s_nop 1" : : "v"(data) : "memory");
}

// With ReLU the int8 result is clamp(rint(v), 0, 127) (NaN -> 0): pack_i8 with lower bound 0.
__device__ __forceinline__ v4i pack_u8_relu(const v4i (&acc)[4], const v4f (&mult)[4]) {
  return pack_i8(acc, mult, 0.0f);
}

// Returns a copy of a kernel-argument struct with every 32-bit word already in an SGPR.
// The compiler otherwise fetches kernel arguments lazily, one s_load batch (and one full
// memory round trip) per first use, and a kernel whose addressing needs many fields pays
// several such round trips before its first global load is issued.  Consuming every word
// in an empty asm statement makes all of them load in one batch at kernel entry.
template <typename T>
__device__ __forceinline__ T preload_args(const T& in) {
  static_assert(sizeof(T) % 4 == 0, "kernel argument structs are made of 32-bit words");
  constexpr int kWords = static_cast<int>(sizeof(T) / 4);
  union {
    T t;
    int w[kWords];
  } u;
  u.t = in;
#pragma unroll
  for (int i = 0; i < kWords; ++i) asm volatile("" : "+s"(u.w[i]));
  return u.t;
}

// 16 bytes from an arbitrary byte offset of an LDS buffer, built from five aligned dword
// reads and byte-funnel shifts (v_alignbyte_b32).  Reads bytes [o & ~3, (o & ~3) + 20).
__device__ __forceinline__ v4i lds_load16_unaligned(const unsigned char* base, int o) {
  const int o4 = o & ~3;
  const unsigned sh = static_cast<unsigned>(o & 3);
  const unsigned* p = reinterpret_cast<const unsigned*>(base + o4);
  const unsigned d0 = p[0], d1 = p[1], d2 = p[2], d3 = p[3], d4 = p[4];
  v4i r;
  r[0] = static_cast<int>(__builtin_amdgcn_alignbyte(d1, d0, sh));
  r[1] = static_cast<int>(__builtin_amdgcn_alignbyte(d2, d1, sh));
  r[2] = static_cast<int>(__builtin_amdgcn_alignbyte(d3, d2, sh));
  r[3] = static_cast<int>(__builtin_amdgcn_alignbyte(d4, d3, sh));
  return r;
}

// Writes one lane's 16 accumulators (channel kc0 + 4*j + r held in acc[j][r]) of one
// output pixel at y + obase.  `ep_bias` / `ep_mult` point at the LDS copies of the bias and
// requantization multiplier of channel kc0 (16 consecutive entries, 16-byte aligned); they
// are read four channels at a time to keep few registers live.  `full`: all 16 channels
// exist and the destination is 16-byte aligned, so vector stores are used; otherwise
// channels at or beyond Kg are skipped.
template <int EPI>
__device__ __forceinline__ void store16(void* y, size_t obase, const v4i (&acc)[4], int kc0, int Kg, bool full,
                                        const int32_t* ep_bias, const float* ep_mult, int relu) {
  if constexpr (EPI == kEpiI8) {
    const float lo = relu ? 0.0f : -128.0f;
    int8_t* yp = static_cast<int8_t*>(y) + obase;
    v4i pk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i bb = reinterpret_cast<const v4i*>(ep_bias)[j];
      const v4f mm = reinterpret_cast<const v4f*>(ep_mult)[j];
      unsigned u = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = requant_i8(acc[j][r], bb[r], mm[r], lo);
        u |= (static_cast<unsigned>(q) & 0xffu) << (8 * r);
        if (!full && kc0 + 4 * j + r < Kg) yp[4 * j + r] = static_cast<int8_t>(q);
      }
      pk[j] = static_cast<int>(u);
    }
    if (full) {
      *reinterpret_cast<v4i*>(yp) = pk;
      store_gap(pk);
    }
  } else if constexpr (EPI == kEpiAcc32) {
    (void)ep_bias;
    (void)ep_mult;
    (void)relu;
    int32_t* yp = static_cast<int32_t*>(y) + obase;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (full) {
        reinterpret_cast<v4i*>(yp)[j] = acc[j];
        store_gap(acc[j]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kc0 + 4 * j + r < Kg) yp[4 * j + r] = acc[j][r];
      }
    }
  } else {
    float* yp = static_cast<float*>(y) + obase;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4i bb = reinterpret_cast<const v4i*>(ep_bias)[j];
      const v4f mm = reinterpret_cast<const v4f*>(ep_mult)[j];
      v4f f;
#pragma unroll
      for (int r = 0; r < 4; ++r) f[r] = dequant_f32(acc[j][r], bb[r], mm[r], relu);
      if (full) {
        reinterpret_cast<v4f*>(yp)[j] = f;
        store_gap(f);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kc0 + 4 * j + r < Kg) yp[4 * j + r] = f[r];
      }
    }
  }
}

// As store16, for accumulators that already include the bias (they were initialised with
// it): requantizes with the per-channel multipliers at `ep_mult` (LDS).
//
// int8: q = clamp(rint(v), lo, 127) computed as rint(med3(v, lo, 127)) - equal because
// the bounds are integers - in four instructions per value: convert, multiply,
// v_med3_f32 (which returns its lower bound, lo, for a NaN input: the NaN rule), and the
// 1.5 * 2^23 addition that rounds; v_perm_b32 gathers the four low bytes.
template <int EPI>
__device__ __forceinline__ void store16_biased(void* y, size_t obase, const v4i& a0, const v4i& a1, const v4i& a2,
                                               const v4i& a3, int kc0, int Kg, bool full, const float* ep_mult,
                                               int relu) {
  const v4i* acc[4] = {&a0, &a1, &a2, &a3};
  if constexpr (EPI == kEpiI8) {
    const float lo = relu ? 0.0f : -128.0f;
    int8_t* yp = static_cast<int8_t*>(y) + obase;
    v4i pk;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4f mm = reinterpret_cast<const v4f*>(ep_mult)[j];
      unsigned u[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = static_cast<float>((*acc[j])[r]) * mm[r];
        u[r] = __float_as_uint(__builtin_amdgcn_fmed3f(v, lo, 127.0f) + 12582912.0f);
      }
      pk[j] = static_cast<int>(__builtin_amdgcn_perm(u[1], u[0], 0x0c0c0400u) |
                               __builtin_amdgcn_perm(u[3], u[2], 0x04000c0cu));
      if (!full) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kc0 + 4 * j + r < Kg) yp[4 * j + r] = static_cast<int8_t>(u[r] & 0xffu);
      }
    }
    if (full) {
      *reinterpret_cast<v4i*>(yp) = pk;
      store_gap(pk);
    }
  } else if constexpr (EPI == kEpiAcc32) {
    (void)ep_mult;
    (void)relu;
    int32_t* yp = static_cast<int32_t*>(y) + obase;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (full) {
        reinterpret_cast<v4i*>(yp)[j] = *acc[j];
        store_gap(*acc[j]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kc0 + 4 * j + r < Kg) yp[4 * j + r] = (*acc[j])[r];
      }
    }
  } else {
    float* yp = static_cast<float*>(y) + obase;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const v4f mm = reinterpret_cast<const v4f*>(ep_mult)[j];
      v4f f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = static_cast<float>((*acc[j])[r]) * mm[r];
        if (relu) v = (v > 0.0f) ? v : 0.0f;
        f[r] = v;
      }
      if (full) {
        reinterpret_cast<v4f*>(yp)[j] = f;
        store_gap(f);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kc0 + 4 * j + r < Kg) yp[4 * j + r] = f[r];
      }
    }
  }
}

// Bias and requantization multiplier of `count` channels starting at kabs (entries at or
// beyond `valid` are 0) into LDS, one channel per thread of the workgroup.
template <int EPI>
__device__ __forceinline__ void stage_requant(const Requant& rq, int kabs, int valid, int count, int32_t* ep_bias,
                                              float* ep_mult) {
  if constexpr (EPI != kEpiAcc32) {
    for (int c = threadIdx.x; c < count; c += blockDim.x) {
      const bool ok = c < valid;
      ep_bias[c] = (ok && rq.bias) ? rq.bias[kabs + c] : 0;
      ep_mult[c] = ok ? requant_multiplier(rq.act_scale, rq.wscale[kabs + c]) : 0.0f;
    }
  }
}

}  // namespace miq
