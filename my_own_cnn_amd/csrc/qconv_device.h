// Device helpers shared by the MFMA convolution kernels: operand types, unaligned LDS
// reads and the fused output stage for one lane's 16 consecutive output channels.
#pragma once

#include "qconv_internal.h"

namespace miq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

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

// Bias and requantization multipliers of channels kabs .. kabs+15 (valid below kc0 < Kg).
template <int EPI>
__device__ __forceinline__ void load_requant16(const Requant& rq, int kc0, int Kg, int kabs, int32_t (&bv)[16],
                                               float (&mv)[16]) {
  if constexpr (EPI != kEpiAcc32) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const bool ok = kc0 + c < Kg;
      bv[c] = (ok && rq.bias) ? rq.bias[kabs + c] : 0;
      mv[c] = ok ? requant_multiplier(rq.act_scale, rq.wscale[kabs + c]) : 0.0f;
    }
  }
}

// Writes one lane's 16 accumulators (channel kc0 + 4*j + r held in acc[j][r]) of one
// output pixel at y + obase.  `full`: all 16 channels exist and the destination is 16-byte
// aligned, so vector stores are used; otherwise channels at or beyond Kg are skipped.
template <int EPI>
__device__ __forceinline__ void store16(void* y, size_t obase, const v4i (&acc)[4], int kc0, int Kg, bool full,
                                        const int32_t (&bv)[16], const float (&mv)[16], int relu) {
  int32_t v[16];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) v[4 * j + r] = acc[j][r];

  if constexpr (EPI == kEpiI8) {
    const float lo = relu ? 0.0f : -128.0f;
    int q[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) q[c] = requant_i8(v[c], bv[c], mv[c], lo);
    int8_t* yp = static_cast<int8_t*>(y) + obase;
    if (full) {
      v4i pk;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const unsigned u = (static_cast<unsigned>(q[4 * d]) & 0xffu) | ((static_cast<unsigned>(q[4 * d + 1]) & 0xffu) << 8) |
                           ((static_cast<unsigned>(q[4 * d + 2]) & 0xffu) << 16) |
                           ((static_cast<unsigned>(q[4 * d + 3]) & 0xffu) << 24);
        pk[d] = static_cast<int>(u);
      }
      *reinterpret_cast<v4i*>(yp) = pk;
    } else {
#pragma unroll
      for (int c = 0; c < 16; ++c)
        if (kc0 + c < Kg) yp[c] = static_cast<int8_t>(q[c]);
    }
  } else if constexpr (EPI == kEpiAcc32) {
    int32_t* yp = static_cast<int32_t*>(y) + obase;
    if (full) {
#pragma unroll
      for (int d = 0; d < 4; ++d) reinterpret_cast<v4i*>(yp)[d] = v4i{v[4 * d], v[4 * d + 1], v[4 * d + 2], v[4 * d + 3]};
    } else {
#pragma unroll
      for (int c = 0; c < 16; ++c)
        if (kc0 + c < Kg) yp[c] = v[c];
    }
  } else {
    float f[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) f[c] = dequant_f32(v[c], bv[c], mv[c], relu);
    float* yp = static_cast<float*>(y) + obase;
    if (full) {
#pragma unroll
      for (int d = 0; d < 4; ++d) reinterpret_cast<v4f*>(yp)[d] = v4f{f[4 * d], f[4 * d + 1], f[4 * d + 2], f[4 * d + 3]};
    } else {
#pragma unroll
      for (int c = 0; c < 16; ++c)
        if (kc0 + c < Kg) yp[c] = f[c];
    }
  }
}

}  // namespace miq
