// C++ drop-in implementations of the reference's GPU entry points for the quantized
// path (conv_quant_detail::launch_*_qi32_{u8,s5}, /root/reference/src/cuda_kernels.cu:1465-1499)
// and of the new int8 launchers, as thin wrappers over the C-ABI.  A non-OK status is
// turned into std::runtime_error carrying the library's message, which is how the
// reference reports shape errors (conv_types.h:125-169) and runtime failures
// (cuda_utils.h:7-13).

#include <cstddef>
#include <stdexcept>
#include <string>

#include "conv_types.h"
#include "miq_qconv.h"

static_assert(sizeof(miq_conv2d_params) == sizeof(Conv2DParams), "Conv2DParams layout");
static_assert(offsetof(miq_conv2d_params, groups) == offsetof(Conv2DParams, groups), "Conv2DParams layout");
static_assert(sizeof(miq_block_conv2d_params) == sizeof(BlockConv2DParams), "BlockConv2DParams layout");
static_assert(offsetof(miq_block_conv2d_params, block_bx) == offsetof(BlockConv2DParams, block_bx),
              "BlockConv2DParams layout");
static_assert(sizeof(miq_qparams_u8) == sizeof(nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>),
              "U8 qparams layout");
static_assert(sizeof(miq_qparams_s5) == sizeof(nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>),
              "S5 qparams layout");

namespace {

using U8 = nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>;
using S5 = nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>;

void throw_on_error(int status, const char* entry) {
  if (status != MIQ_OK) {
    throw std::runtime_error(std::string(entry) + ": " + miq_last_error_message() + " (" +
                             miq_status_string(status) + ")");
  }
}

miq_conv2d_params to_c(const Conv2DParams& p) {
  return miq_conv2d_params{p.pad_h, p.pad_w, p.stride_h, p.stride_w, p.dilation_h, p.dilation_w, p.groups};
}

miq_block_conv2d_params to_c(const BlockConv2DParams& p) {
  return miq_block_conv2d_params{to_c(p.conv), p.block_by, p.block_bx};
}

miq_qconv_desc make_desc(int n, int h, int w, int c, int r, int s, int k, const Conv2DParams& p, bool relu,
                         float in_scale, float out_scale) {
  miq_qconv_desc d{};
  d.n = n; d.h = h; d.w = w; d.c = c;
  d.k = k; d.r = r; d.s = s;
  d.conv = to_c(p);
  d.relu = relu ? 1 : 0;
  d.in_scale = in_scale;
  d.out_scale = out_scale;
  d.algo = MIQ_ALGO_AUTO;
  return d;
}

}  // namespace

void launch_fprop_nhwc(const float* d_x, const float* d_w, float* d_y, int n, int h, int w, int c, int r, int s,
                       int k, const Conv2DParams& p) {
  const miq_conv2d_params cp = to_c(p);
  throw_on_error(miq_fprop_nhwc_f32(d_x, d_w, d_y, n, h, w, c, r, s, k, &cp, MIQ_ALGO_AUTO, nullptr),
                 "launch_fprop_nhwc");
}

void launch_bprop_nhwc(const float* d_dy, const float* d_w, float* d_dx, int n, int h, int w, int c, int r, int s,
                       int k, const Conv2DParams& p) {
  const miq_conv2d_params cp = to_c(p);
  throw_on_error(miq_bprop_nhwc_f32(d_dy, d_w, d_dx, n, h, w, c, r, s, k, &cp, MIQ_ALGO_AUTO, nullptr),
                 "launch_bprop_nhwc");
}

void launch_grad_nhwc(const float* d_x, const float* d_dy, float* d_dw, int n, int h, int w, int c, int r, int s,
                      int k, const Conv2DParams& p) {
  const miq_conv2d_params cp = to_c(p);
  throw_on_error(miq_grad_nhwc_f32(d_x, d_dy, d_dw, n, h, w, c, r, s, k, &cp, MIQ_ALGO_AUTO, nullptr),
                 "launch_grad_nhwc");
}

void launch_block_fprop_nhwc(const float* d_x, const float* d_w, float* d_y, int n, int h, int w, int c, int r, int s,
                             int k, const BlockConv2DParams& p, const float* d_bias, BlockBiasMode bias_mode) {
  const miq_block_conv2d_params bp = to_c(p);
  throw_on_error(miq_block_fprop_nhwc_f32(d_x, d_w, d_y, n, h, w, c, r, s, k, &bp, d_bias,
                                          static_cast<int32_t>(bias_mode), MIQ_ALGO_AUTO, nullptr),
                 "launch_block_fprop_nhwc");
}

void launch_block_bprop_nhwc(const float* d_dy, const float* d_w, float* d_dx, int n, int h, int w, int c, int r,
                             int s, int k, const BlockConv2DParams& p) {
  const miq_block_conv2d_params bp = to_c(p);
  throw_on_error(miq_block_bprop_nhwc_f32(d_dy, d_w, d_dx, n, h, w, c, r, s, k, &bp, MIQ_ALGO_AUTO, nullptr),
                 "launch_block_bprop_nhwc");
}

void launch_block_grad_nhwc(const float* d_x, const float* d_dy, float* d_dw, int n, int h, int w, int c, int r, int s,
                            int k, const BlockConv2DParams& p, float* d_dbias, BlockBiasMode bias_mode) {
  const miq_block_conv2d_params bp = to_c(p);
  throw_on_error(miq_block_grad_nhwc_f32(d_x, d_dy, d_dw, n, h, w, c, r, s, k, &bp, d_dbias,
                                         static_cast<int32_t>(bias_mode), MIQ_ALGO_AUTO, nullptr),
                 "launch_block_grad_nhwc");
}

namespace conv_quant_detail {

void launch_fprop_nhwc_qi32_u8(const float* d_x, const float* d_w, int32_t* d_y, int n, int h, int w, int c, int r,
                               int s, int k, const Conv2DParams& p, const U8* in_qp, const U8* f_qp) {
  const miq_conv2d_params cp = to_c(p);
  throw_on_error(miq_fprop_nhwc_qi32_u8(d_x, d_w, d_y, n, h, w, c, r, s, k, &cp,
                                        reinterpret_cast<const miq_qparams_u8*>(in_qp),
                                        reinterpret_cast<const miq_qparams_u8*>(f_qp), nullptr),
                 "launch_fprop_nhwc_qi32_u8");
}

void launch_fprop_nhwc_qi32_s5(const float* d_x, const float* d_w, int32_t* d_y, int n, int h, int w, int c, int r,
                               int s, int k, const Conv2DParams& p, const S5* in_qp, const S5* f_qp) {
  const miq_conv2d_params cp = to_c(p);
  throw_on_error(miq_fprop_nhwc_qi32_s5(d_x, d_w, d_y, n, h, w, c, r, s, k, &cp,
                                        reinterpret_cast<const miq_qparams_s5*>(in_qp),
                                        reinterpret_cast<const miq_qparams_s5*>(f_qp), nullptr),
                 "launch_fprop_nhwc_qi32_s5");
}

void launch_block_fprop_nhwc_qi32_u8(const float* d_x, const float* d_w, int32_t* d_y, int n, int h, int w, int c,
                                     int r, int s, int k, const BlockConv2DParams& p, const U8* in_qp, const U8* f_qp) {
  const miq_block_conv2d_params cp = to_c(p);
  throw_on_error(miq_block_fprop_nhwc_qi32_u8(d_x, d_w, d_y, n, h, w, c, r, s, k, &cp,
                                              reinterpret_cast<const miq_qparams_u8*>(in_qp),
                                              reinterpret_cast<const miq_qparams_u8*>(f_qp), nullptr),
                 "launch_block_fprop_nhwc_qi32_u8");
}

void launch_block_fprop_nhwc_qi32_s5(const float* d_x, const float* d_w, int32_t* d_y, int n, int h, int w, int c,
                                     int r, int s, int k, const BlockConv2DParams& p, const S5* in_qp, const S5* f_qp) {
  const miq_block_conv2d_params cp = to_c(p);
  throw_on_error(miq_block_fprop_nhwc_qi32_s5(d_x, d_w, d_y, n, h, w, c, r, s, k, &cp,
                                              reinterpret_cast<const miq_qparams_s5*>(in_qp),
                                              reinterpret_cast<const miq_qparams_s5*>(f_qp), nullptr),
                 "launch_block_fprop_nhwc_qi32_s5");
}

}  // namespace conv_quant_detail

void launch_fprop_nhwc_qi8(const int8_t* d_x, const int8_t* d_w, int8_t* d_y, int n, int h, int w, int c, int r, int s,
                           int k, const Conv2DParams& p, const RequantParams& rq, void* stream) {
  const miq_qconv_desc d = make_desc(n, h, w, c, r, s, k, p, rq.relu, rq.in_scale, rq.out_scale);
  throw_on_error(miq_qconv2d_nhwc_i8(&d, d_x, d_w, rq.d_bias, rq.d_w_scale, d_y, stream), "launch_fprop_nhwc_qi8");
}

void launch_fprop_nhwc_qi8_acc32(const int8_t* d_x, const int8_t* d_w, int32_t* d_y, int n, int h, int w, int c, int r,
                                 int s, int k, const Conv2DParams& p, void* stream) {
  const miq_qconv_desc d = make_desc(n, h, w, c, r, s, k, p, false, 1.f, 1.f);
  throw_on_error(miq_qconv2d_nhwc_i8_acc32(&d, d_x, d_w, d_y, stream), "launch_fprop_nhwc_qi8_acc32");
}

void launch_fprop_nhwc_qi8_dequant(const int8_t* d_x, const int8_t* d_w, float* d_y, int n, int h, int w, int c, int r,
                                   int s, int k, const Conv2DParams& p, const RequantParams& rq, void* stream) {
  const miq_qconv_desc d = make_desc(n, h, w, c, r, s, k, p, rq.relu, rq.in_scale, rq.out_scale);
  throw_on_error(miq_qconv2d_nhwc_i8_dequant(&d, d_x, d_w, rq.d_bias, rq.d_w_scale, d_y, stream),
                 "launch_fprop_nhwc_qi8_dequant");
}
