// Quantization parameter types of the quantized NHWC convolution path.
//
// Drop-in surface: the enumerators, the QuantizationParameters<> specialisations,
// getZeroPoint and the supported-input trait declare exactly what
// /root/reference/src/nnalgebra_quantization.h:15-93 declares, so that code written
// against the reference (quant_conv_test.cu, cpu_ref.cpp) compiles and links against
// this library unchanged.  The structs are copied to the device byte-for-byte by the
// reference's callers (quant_conv_test.cu:150-151), so their layouts are pinned below.
//
// Addition (not in the reference): DataType::LinQuantI8, appended after LinQuantI32 so
// that every existing enumerator keeps its value.  It describes symmetric signed int8
// codes (zero point 0) with one float scale; the native int8 entry points use it.
#pragma once

#include <cstddef>
#include <cstdint>
#include <type_traits>

#if !defined(__HIPCC__) && !defined(__CUDACC__)
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif

using real32_t = float;

namespace nnalgebra {

// Enumerator order and values follow nnalgebra_quantization.h:19-24; LinQuantI8 is new.
enum class DataType : int {
  Real32,
  LinQuantU8,
  LinQuantS5,
  LinQuantI32,
  LinQuantI8,
};

template <DataType T>
struct QuantizationParameters;

// uint8 codes with an affine zero point (nnalgebra_quantization.h:29-34).
template <>
struct QuantizationParameters<DataType::LinQuantU8> {
  uint8_t zero_point = 0;
  real32_t scale = 1.f;
  bool symmetric = false;
};

// 5-bit signed codes (nnalgebra_quantization.h:36-41).
template <>
struct QuantizationParameters<DataType::LinQuantS5> {
  int8_t zero_point = 0;
  uint8_t n_bins = 0;
  real32_t scale = 1.f;
};

// int32 accumulators; the zero point is fixed at 0 (nnalgebra_quantization.h:43-47).
template <>
struct QuantizationParameters<DataType::LinQuantI32> {
  static constexpr int32_t zero_point = 0;
  real32_t scale = 1.f;
};

// float codes (nnalgebra_quantization.h:49-54).
template <>
struct QuantizationParameters<DataType::Real32> {
  uint16_t zero_point = 0;
  real32_t scale = 1.f;
  bool symmetric = false;
};

// New: symmetric signed int8 codes.  The native int8 convolution requires
// zero_point == 0 (activations and weights are symmetric); scale is the real value
// of one code step.
template <>
struct QuantizationParameters<DataType::LinQuantI8> {
  int8_t zero_point = 0;
  real32_t scale = 1.f;
};

// Layouts the device side relies on (structs are memcpy'd raw to the GPU).
static_assert(sizeof(QuantizationParameters<DataType::LinQuantU8>) == 12, "U8 qparams layout");
static_assert(offsetof(QuantizationParameters<DataType::LinQuantU8>, zero_point) == 0, "U8 zero_point offset");
static_assert(offsetof(QuantizationParameters<DataType::LinQuantU8>, scale) == 4, "U8 scale offset");
static_assert(offsetof(QuantizationParameters<DataType::LinQuantU8>, symmetric) == 8, "U8 symmetric offset");
static_assert(sizeof(QuantizationParameters<DataType::LinQuantS5>) == 8, "S5 qparams layout");
static_assert(offsetof(QuantizationParameters<DataType::LinQuantS5>, zero_point) == 0, "S5 zero_point offset");
static_assert(offsetof(QuantizationParameters<DataType::LinQuantS5>, n_bins) == 1, "S5 n_bins offset");
static_assert(offsetof(QuantizationParameters<DataType::LinQuantS5>, scale) == 4, "S5 scale offset");
static_assert(sizeof(QuantizationParameters<DataType::LinQuantI32>) == 4, "I32 qparams layout");
static_assert(sizeof(QuantizationParameters<DataType::LinQuantI8>) == 8, "I8 qparams layout");

// Zero point as an int, per type (nnalgebra_quantization.h:56-81).
template <DataType T>
__host__ __device__ inline int getZeroPoint(const QuantizationParameters<T>& qp);

template <>
__host__ __device__ inline int getZeroPoint<DataType::LinQuantU8>(
    const QuantizationParameters<DataType::LinQuantU8>& qp) {
  return static_cast<int>(qp.zero_point);
}

template <>
__host__ __device__ inline int getZeroPoint<DataType::LinQuantS5>(
    const QuantizationParameters<DataType::LinQuantS5>& qp) {
  return static_cast<int>(qp.zero_point);
}

template <>
__host__ __device__ inline int getZeroPoint<DataType::LinQuantI32>(
    const QuantizationParameters<DataType::LinQuantI32>&) {
  return 0;
}

template <>
__host__ __device__ inline int getZeroPoint<DataType::Real32>(
    const QuantizationParameters<DataType::Real32>& qp) {
  return static_cast<int>(qp.zero_point);
}

template <>
__host__ __device__ inline int getZeroPoint<DataType::LinQuantI8>(
    const QuantizationParameters<DataType::LinQuantI8>& qp) {
  return static_cast<int>(qp.zero_point);
}

// Which code types the int32-accumulator convolutions accept
// (nnalgebra_quantization.h:83-93).  LinQuantI8 has its own entry points and is
// deliberately not added here, so the qi32 templates keep their exact contract.
template <DataType T>
struct IsSupportedQuantizedInput : std::false_type {};

template <>
struct IsSupportedQuantizedInput<DataType::LinQuantU8> : std::true_type {};

template <>
struct IsSupportedQuantizedInput<DataType::LinQuantS5> : std::true_type {};

template <DataType T>
inline constexpr bool kIsSupportedQuantizedInput = IsSupportedQuantizedInput<T>::value;

}  // namespace nnalgebra
