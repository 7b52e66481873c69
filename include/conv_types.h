// C++ drop-in surface of the quantized NHWC convolution path.
//
// The descriptors, shape inference, index helpers, the conv_quant_detail declarations
// and the four dispatch templates declare what /root/reference/src/conv_types.h:21-202
// and :213-342 declare for this path, with the same names, members, defaults and
// signatures, so that callers written against the reference (quant_conv_test.cu and the
// verify_tensors / benchmark_cuda_op harness) compile unchanged and resolve to this
// library's implementations.  The fp32 launchers launch_{,block_}{fprop,bprop,grad}_nhwc and the
// CPU functions cpu_{,block_}{fprop,bprop,grad}_nhwc are declared as the reference declares
// them (conv_types.h:204-212, :287-304); this library defines the launchers and no CPU
// convolution (the CPU functions are the reference's cpu_ref.cpp, or the test oracle's
// adapter).  The cuDNN comparison functions of the reference header are not part of this
// build and are not declared here.
//
// Additions beside the reference surface (nothing existing changes):
//   * RequantParams and the native int8 launchers launch_fprop_nhwc_qi8{,_acc32,_dequant}
//   * an optional trailing hipStream_t-as-void* argument on the new launchers
//   * benchmark_hip_op, the HIP-named alias of benchmark_cuda_op
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "nnalgebra_quantization.h"

// Convolution hyper-parameters (conv_types.h:21-29).
struct Conv2DParams {
  int pad_h = 1;
  int pad_w = 1;
  int stride_h = 1;
  int stride_w = 1;
  int dilation_h = 1;
  int dilation_w = 1;
  int groups = 1;
};

// Blocked ("locally shared") convolution: the output plane is cut into block_by x block_bx
// blocks, each with its own filter (conv_types.h:31-35).
struct BlockConv2DParams {
  Conv2DParams conv;
  int block_by = 1;
  int block_bx = 1;
};

static_assert(sizeof(Conv2DParams) == 28, "Conv2DParams is memcpy-compatible with miq_conv2d_params");
static_assert(sizeof(BlockConv2DParams) == 36, "BlockConv2DParams is memcpy-compatible with miq_block_conv2d_params");

// Bias sharing of the blocked fp32 path (conv_types.h:37-40); kept for descriptor parity.
enum class BlockBiasMode {
  PerBlock = 0,
  Shared = 1,
};

// Host tensor of quantized codes stored as float, NHWC (conv_types.h:42-55).
struct TensorNHWC {
  int n = 0;
  int h = 0;
  int w = 0;
  int c = 0;
  std::vector<float> data;

  TensorNHWC() = default;
  TensorNHWC(int n_, int h_, int w_, int c_)
      : n(n_), h(h_), w(w_), c(c_), data(static_cast<size_t>(n_) * h_ * w_ * c_) {}

  size_t elements() const { return static_cast<size_t>(n) * h * w * c; }
  float* ptr() { return data.data(); }
  const float* ptr() const { return data.data(); }
};

// Filter, output-channel major [K, R, S, C/groups] (conv_types.h:57-71).
struct FilterKRSC {
  int r = 0;
  int s = 0;
  int cin_per_group = 0;
  int k = 0;
  std::vector<float> data;

  FilterKRSC() = default;
  FilterKRSC(int r_, int s_, int cin_per_group_, int k_)
      : r(r_), s(s_), cin_per_group(cin_per_group_), k(k_),
        data(static_cast<size_t>(r_) * s_ * cin_per_group_ * k_) {}

  size_t elements() const { return static_cast<size_t>(r) * s * cin_per_group * k; }
  float* ptr() { return data.data(); }
  const float* ptr() const { return data.data(); }
};

using FilterHWCN = FilterKRSC;

// Blocked filter [K, By, Bx, R, S, C/groups] (conv_types.h:75-93).
struct BlockFilterKByBxRSC {
  int k = 0;
  int by = 0;
  int bx = 0;
  int r = 0;
  int s = 0;
  int cin_per_group = 0;
  std::vector<float> data;

  BlockFilterKByBxRSC() = default;
  BlockFilterKByBxRSC(int k_, int by_, int bx_, int r_, int s_, int cin_per_group_)
      : k(k_), by(by_), bx(bx_), r(r_), s(s_), cin_per_group(cin_per_group_),
        data(static_cast<size_t>(k_) * by_ * bx_ * r_ * s_ * cin_per_group_) {}

  size_t elements() const { return static_cast<size_t>(k) * by * bx * r * s * cin_per_group; }
  float* ptr() { return data.data(); }
  const float* ptr() const { return data.data(); }
};

// int32 accumulator tensor, NHWC (conv_types.h:95-110).
struct TensorNHWCI32 {
  int n = 0;
  int h = 0;
  int w = 0;
  int c = 0;
  std::vector<int32_t> data;

  TensorNHWCI32() = default;
  TensorNHWCI32(int n_, int h_, int w_, int c_)
      : n(n_), h(h_), w(w_), c(c_), data(static_cast<size_t>(n_) * h_ * w_ * c_) {}

  size_t elements() const { return static_cast<size_t>(n) * h * w * c; }
  int32_t* ptr() { return data.data(); }
  const int32_t* ptr() const { return data.data(); }
};

struct ConvShape {
  int ho = 0;
  int wo = 0;
  int cin_group = 0;
  int kout_group = 0;
};

struct BlockConvShape {
  ConvShape base;
  int block_ho = 0;
  int block_wo = 0;
};

// Output geometry with the reference's validation rules and messages
// (conv_types.h:125-146).
inline ConvShape infer_conv_shape(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p) {
  if (p.groups <= 0) throw std::runtime_error("groups must be > 0");
  if (x.c % p.groups != 0) throw std::runtime_error("input channels must be divisible by groups");
  if (w.k % p.groups != 0) throw std::runtime_error("output channels must be divisible by groups");
  ConvShape out;
  out.cin_group = x.c / p.groups;
  if (out.cin_group != w.cin_per_group) throw std::runtime_error("filter cin_per_group mismatch");

  const int rows = x.h + 2 * p.pad_h - p.dilation_h * (w.r - 1) - 1;
  const int cols = x.w + 2 * p.pad_w - p.dilation_w * (w.s - 1) - 1;
  if (rows < 0 || cols < 0) throw std::runtime_error("invalid output size (negative numerator)");
  if (p.stride_h <= 0 || p.stride_w <= 0) throw std::runtime_error("stride must be > 0");
  out.ho = rows / p.stride_h + 1;
  out.wo = cols / p.stride_w + 1;
  if (out.ho <= 0 || out.wo <= 0) throw std::runtime_error("computed output size is <= 0");
  out.kout_group = w.k / p.groups;
  return out;
}

// Blocked geometry (conv_types.h:148-169).
inline BlockConvShape infer_block_conv_shape(const TensorNHWC& x, const BlockFilterKByBxRSC& w,
                                             const BlockConv2DParams& p) {
  if (p.block_by <= 0 || p.block_bx <= 0) throw std::runtime_error("block_by and block_bx must be > 0");
  if (w.by != p.block_by || w.bx != p.block_bx) throw std::runtime_error("blocked filter block grid mismatch");
  BlockConvShape out;
  out.base = infer_conv_shape(x, FilterKRSC(w.r, w.s, w.cin_per_group, w.k), p.conv);
  if (out.base.ho % p.block_by != 0 || out.base.wo % p.block_bx != 0) {
    throw std::runtime_error("blocked convolution requires Ho/Wo divisible by block grid");
  }
  out.block_ho = out.base.ho / p.block_by;
  out.block_wo = out.base.wo / p.block_bx;
  return out;
}

// Linear offsets of the three layouts (conv_types.h:171-188).
__host__ __device__ inline size_t idx_nhwc(int n, int h, int w, int c, int H, int W, int C) {
  return ((static_cast<size_t>(n) * H + h) * W + w) * C + c;
}

__host__ __device__ inline size_t idx_krsc(int k, int r, int s, int c, int R, int S, int C) {
  return ((static_cast<size_t>(k) * R + r) * S + s) * C + c;
}

__host__ __device__ inline size_t idx_kbybxrsc(int k, int by, int bx, int r, int s, int c,
                                               int By, int Bx, int R, int S, int C) {
  return ((((static_cast<size_t>(k) * By + by) * Bx + bx) * R + r) * S + s) * C + c;
}

__host__ __device__ inline size_t idx_block_bias(int k, int by, int bx, int by_count, int bx_count,
                                                 BlockBiasMode mode) {
  const bool per_block = (mode == BlockBiasMode::PerBlock);
  return (static_cast<size_t>(k) * by_count + (per_block ? by : 0)) * bx_count + (per_block ? bx : 0);
}

struct VerifyResult {
  float max_abs_err = 0.0f;
  float max_rel_err = 0.0f;
  size_t max_abs_idx = 0;
  size_t max_rel_idx = 0;
  bool passed = false;
};

struct BenchResult {
  float median_ms = 0.0f;
  float p90_ms = 0.0f;
  float gflops = 0.0f;
};

// fp32 CPU reference path (conv_types.h:204-212): declared for callers written against the
// reference; defined by the reference's cpu_ref.cpp (or by this repository's test oracle).
void cpu_fprop_nhwc(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p, TensorNHWC& y);
void cpu_bprop_nhwc(const TensorNHWC& dy, const FilterKRSC& w, const Conv2DParams& p, TensorNHWC& dx);
void cpu_grad_nhwc(const TensorNHWC& x, const TensorNHWC& dy, const Conv2DParams& p, FilterKRSC& dw);
void cpu_block_fprop_nhwc(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p, TensorNHWC& y,
                          const float* bias = nullptr, BlockBiasMode bias_mode = BlockBiasMode::PerBlock);
void cpu_block_bprop_nhwc(const TensorNHWC& dy, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p, TensorNHWC& dx);
void cpu_block_grad_nhwc(const TensorNHWC& x, const TensorNHWC& dy, const BlockConv2DParams& p, BlockFilterKByBxRSC& dw,
                         float* dbias = nullptr, BlockBiasMode bias_mode = BlockBiasMode::PerBlock);

namespace conv_quant_detail {

// CPU reference path (conv_types.h:215-230).  Defined by the reference's cpu_ref.cpp (or
// by this repository's test oracle); this library itself contains no CPU convolution.
void cpu_fprop_nhwc_qi32_u8(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p,
                            TensorNHWCI32& y,
                            const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* in_qp,
                            const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* f_qp);
void cpu_fprop_nhwc_qi32_s5(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p,
                            TensorNHWCI32& y,
                            const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* in_qp,
                            const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* f_qp);
void cpu_block_fprop_nhwc_qi32_u8(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p,
                                  TensorNHWCI32& y,
                                  const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* in_qp,
                                  const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* f_qp);
void cpu_block_fprop_nhwc_qi32_s5(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p,
                                  TensorNHWCI32& y,
                                  const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* in_qp,
                                  const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* f_qp);

// GPU path (conv_types.h:232-251), implemented by this library on the default stream.
// All pointers are device pointers; in_qp holds n structs (one per sample).
void launch_fprop_nhwc_qi32_u8(const float* d_x, const float* d_w, int32_t* d_y,
                               int n, int h, int w, int c, int r, int s, int k,
                               const Conv2DParams& p,
                               const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* in_qp,
                               const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* f_qp);
void launch_fprop_nhwc_qi32_s5(const float* d_x, const float* d_w, int32_t* d_y,
                               int n, int h, int w, int c, int r, int s, int k,
                               const Conv2DParams& p,
                               const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* in_qp,
                               const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* f_qp);
void launch_block_fprop_nhwc_qi32_u8(const float* d_x, const float* d_w, int32_t* d_y,
                                     int n, int h, int w, int c, int r, int s, int k,
                                     const BlockConv2DParams& p,
                                     const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* in_qp,
                                     const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>* f_qp);
void launch_block_fprop_nhwc_qi32_s5(const float* d_x, const float* d_w, int32_t* d_y,
                                     int n, int h, int w, int c, int r, int s, int k,
                                     const BlockConv2DParams& p,
                                     const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* in_qp,
                                     const nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>* f_qp);

}  // namespace conv_quant_detail

// Type-dispatching front ends (conv_types.h:255-285, :308-340): compile-time type gate,
// null-parameter check, then the _u8 / _s5 implementation.
template <nnalgebra::DataType Tin>
inline void cpu_fprop_nhwc_qi32(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p,
                                TensorNHWCI32& y,
                                const nnalgebra::QuantizationParameters<Tin>* in_qp,
                                const nnalgebra::QuantizationParameters<Tin>* f_qp) {
  static_assert(nnalgebra::kIsSupportedQuantizedInput<Tin>,
                "cpu_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5");
  if (in_qp == nullptr || f_qp == nullptr) {
    throw std::runtime_error("quantized CPU fprop requires non-null quantization parameters");
  }
  if constexpr (Tin == nnalgebra::DataType::LinQuantU8) {
    conv_quant_detail::cpu_fprop_nhwc_qi32_u8(x, w, p, y, in_qp, f_qp);
  } else {
    conv_quant_detail::cpu_fprop_nhwc_qi32_s5(x, w, p, y, in_qp, f_qp);
  }
}

template <nnalgebra::DataType Tin>
inline void cpu_block_fprop_nhwc_qi32(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p,
                                      TensorNHWCI32& y,
                                      const nnalgebra::QuantizationParameters<Tin>* in_qp,
                                      const nnalgebra::QuantizationParameters<Tin>* f_qp) {
  static_assert(nnalgebra::kIsSupportedQuantizedInput<Tin>,
                "cpu_block_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5");
  if (in_qp == nullptr || f_qp == nullptr) {
    throw std::runtime_error("quantized blocked CPU fprop requires non-null quantization parameters");
  }
  if constexpr (Tin == nnalgebra::DataType::LinQuantU8) {
    conv_quant_detail::cpu_block_fprop_nhwc_qi32_u8(x, w, p, y, in_qp, f_qp);
  } else {
    conv_quant_detail::cpu_block_fprop_nhwc_qi32_s5(x, w, p, y, in_qp, f_qp);
  }
}

template <nnalgebra::DataType Tin>
inline void launch_fprop_nhwc_qi32(const float* d_x, const float* d_w, int32_t* d_y,
                                   int n, int h, int w, int c, int r, int s, int k,
                                   const Conv2DParams& p,
                                   const nnalgebra::QuantizationParameters<Tin>* in_qp,
                                   const nnalgebra::QuantizationParameters<Tin>* f_qp) {
  static_assert(nnalgebra::kIsSupportedQuantizedInput<Tin>,
                "launch_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5");
  if (in_qp == nullptr || f_qp == nullptr) {
    throw std::runtime_error("quantized CUDA fprop requires non-null quantization parameters");
  }
  if constexpr (Tin == nnalgebra::DataType::LinQuantU8) {
    conv_quant_detail::launch_fprop_nhwc_qi32_u8(d_x, d_w, d_y, n, h, w, c, r, s, k, p, in_qp, f_qp);
  } else {
    conv_quant_detail::launch_fprop_nhwc_qi32_s5(d_x, d_w, d_y, n, h, w, c, r, s, k, p, in_qp, f_qp);
  }
}

template <nnalgebra::DataType Tin>
inline void launch_block_fprop_nhwc_qi32(const float* d_x, const float* d_w, int32_t* d_y,
                                         int n, int h, int w, int c, int r, int s, int k,
                                         const BlockConv2DParams& p,
                                         const nnalgebra::QuantizationParameters<Tin>* in_qp,
                                         const nnalgebra::QuantizationParameters<Tin>* f_qp) {
  static_assert(nnalgebra::kIsSupportedQuantizedInput<Tin>,
                "launch_block_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5");
  if (in_qp == nullptr || f_qp == nullptr) {
    throw std::runtime_error("quantized blocked CUDA fprop requires non-null quantization parameters");
  }
  if constexpr (Tin == nnalgebra::DataType::LinQuantU8) {
    conv_quant_detail::launch_block_fprop_nhwc_qi32_u8(d_x, d_w, d_y, n, h, w, c, r, s, k, p, in_qp, f_qp);
  } else {
    conv_quant_detail::launch_block_fprop_nhwc_qi32_s5(d_x, d_w, d_y, n, h, w, c, r, s, k, p, in_qp, f_qp);
  }
}

// ---- native int8 surface (new; no reference counterpart) ---------------------------

// Requantization inputs of one convolution.  Device pointers: d_bias int32[K] (may be
// null) and d_w_scale float[K].  The arithmetic is defined in miq_qconv.h.
struct RequantParams {
  const int32_t* d_bias = nullptr;
  const float* d_w_scale = nullptr;
  float in_scale = 1.f;
  float out_scale = 1.f;
  bool relu = false;
};

// fp32 convolution, the reference's launch_fprop_nhwc (/root/reference/src/conv_types.h:287-289,
// cuda_kernels.cu:767-823): same signature and meaning, default stream, asynchronous.
void launch_fprop_nhwc(const float* d_x, const float* d_w, float* d_y,
                       int n, int h, int w, int c, int r, int s, int k,
                       const Conv2DParams& p);
// dx and dw of the fp32 convolution, the reference's launch_bprop_nhwc / launch_grad_nhwc
// (conv_types.h:290-295, cuda_kernels.cu:825-937): same signatures and meaning.
void launch_bprop_nhwc(const float* d_dy, const float* d_w, float* d_dx,
                       int n, int h, int w, int c, int r, int s, int k,
                       const Conv2DParams& p);
void launch_grad_nhwc(const float* d_x, const float* d_dy, float* d_dw,
                      int n, int h, int w, int c, int r, int s, int k,
                      const Conv2DParams& p);
// The blocked fp32 convolution, its dx and its dw (+ bias gradient), the reference's
// launch_block_{fprop,bprop,grad}_nhwc (conv_types.h:296-304, cuda_kernels.cu:939-1136): same
// signatures, defaults and meaning.  The bias gradient is the sum of dy over every position of
// the block, as the reference's launcher computes it, in a fixed order.
void launch_block_fprop_nhwc(const float* d_x, const float* d_w, float* d_y,
                             int n, int h, int w, int c, int r, int s, int k,
                             const BlockConv2DParams& p,
                             const float* d_bias = nullptr, BlockBiasMode bias_mode = BlockBiasMode::PerBlock);
void launch_block_bprop_nhwc(const float* d_dy, const float* d_w, float* d_dx,
                             int n, int h, int w, int c, int r, int s, int k,
                             const BlockConv2DParams& p);
void launch_block_grad_nhwc(const float* d_x, const float* d_dy, float* d_dw,
                            int n, int h, int w, int c, int r, int s, int k,
                            const BlockConv2DParams& p,
                            float* d_dbias = nullptr, BlockBiasMode bias_mode = BlockBiasMode::PerBlock);

// y (int8 NHWC) = requant(conv(x, w)); x int8 NHWC, w int8 KRSC, all device pointers.
void launch_fprop_nhwc_qi8(const int8_t* d_x, const int8_t* d_w, int8_t* d_y,
                           int n, int h, int w, int c, int r, int s, int k,
                           const Conv2DParams& p, const RequantParams& rq, void* stream = nullptr);

// Raw int32 accumulators of the int8 convolution.
void launch_fprop_nhwc_qi8_acc32(const int8_t* d_x, const int8_t* d_w, int32_t* d_y,
                                 int n, int h, int w, int c, int r, int s, int k,
                                 const Conv2DParams& p, void* stream = nullptr);

// Dequantized fp32 view of the requantization input.
void launch_fprop_nhwc_qi8_dequant(const int8_t* d_x, const int8_t* d_w, float* d_y,
                                   int n, int h, int w, int c, int r, int s, int k,
                                   const Conv2DParams& p, const RequantParams& rq, void* stream = nullptr);

// ---- harness (conv_types.h:342-348) --------------------------------------------------

// Element-wise comparison with the reference's pass rule (src/verify.cpp:7-36).
VerifyResult verify_tensors(const std::vector<float>& ref, const std::vector<float>& got, float abs_eps, float rel_eps);

// Warmup, then per-iteration HIP-event timing; median / p90 / GFLOP/s (src/bench.cpp:8-45).
BenchResult benchmark_cuda_op(const std::string& op_name,
                              int warmup,
                              int iters,
                              size_t flops,
                              const std::function<void()>& fn);

inline BenchResult benchmark_hip_op(const std::string& op_name, int warmup, int iters, size_t flops,
                                    const std::function<void()>& fn) {
  return benchmark_cuda_op(op_name, warmup, iters, flops, fn);
}
