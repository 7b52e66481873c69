// conv_quant_detail::cpu_*_qi32_{u8,s5} for the test programs, on top of the C oracle
// (oracle/qconv_oracle.c).  TEST INFRASTRUCTURE ONLY: it plays the part of the reference's
// cpu_ref.cpp (/root/reference/src/cpu_ref.cpp:371-401) so that quant_conv_test can be
// re-expressed without the reference's sources.

#include <stdexcept>
#include <vector>

#include "conv_types.h"
#include "qconv_oracle.h"

namespace {

template <nnalgebra::DataType T>
std::vector<int32_t> zero_points(const nnalgebra::QuantizationParameters<T>* qp, int n) {
  std::vector<int32_t> zp(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) zp[static_cast<size_t>(i)] = nnalgebra::getZeroPoint(qp[i]);
  return zp;
}

void conv7(const Conv2DParams& p, int32_t out[7]) {
  out[0] = p.pad_h; out[1] = p.pad_w; out[2] = p.stride_h; out[3] = p.stride_w;
  out[4] = p.dilation_h; out[5] = p.dilation_w; out[6] = p.groups;
}

template <nnalgebra::DataType T>
void regular(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p, TensorNHWCI32& y,
             const nnalgebra::QuantizationParameters<T>* in_qp, const nnalgebra::QuantizationParameters<T>* f_qp) {
  const ConvShape sh = infer_conv_shape(x, w, p);
  y = TensorNHWCI32(x.n, sh.ho, sh.wo, w.k);
  int32_t cv[7];
  conv7(p, cv);
  const auto zp = zero_points(in_qp, x.n);
  if (orc_conv_qi32(x.ptr(), x.n, x.h, x.w, x.c, w.ptr(), w.r, w.s, w.k, cv, zp.data(), nnalgebra::getZeroPoint(*f_qp),
                    0, 0, y.ptr()) != 0) {
    throw std::runtime_error("oracle rejected the shape");
  }
}

template <nnalgebra::DataType T>
void blocked(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p, TensorNHWCI32& y,
             const nnalgebra::QuantizationParameters<T>* in_qp, const nnalgebra::QuantizationParameters<T>* f_qp) {
  const BlockConvShape sh = infer_block_conv_shape(x, w, p);
  y = TensorNHWCI32(x.n, sh.base.ho, sh.base.wo, w.k);
  int32_t cv[7];
  conv7(p.conv, cv);
  const auto zp = zero_points(in_qp, x.n);
  if (orc_conv_qi32(x.ptr(), x.n, x.h, x.w, x.c, w.ptr(), w.r, w.s, w.k, cv, zp.data(), nnalgebra::getZeroPoint(*f_qp),
                    p.block_by, p.block_bx, y.ptr()) != 0) {
    throw std::runtime_error("oracle rejected the shape");
  }
}

}  // namespace

namespace conv_quant_detail {

using U8 = nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantU8>;
using S5 = nnalgebra::QuantizationParameters<nnalgebra::DataType::LinQuantS5>;

void cpu_fprop_nhwc_qi32_u8(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p, TensorNHWCI32& y,
                            const U8* in_qp, const U8* f_qp) {
  regular(x, w, p, y, in_qp, f_qp);
}
void cpu_fprop_nhwc_qi32_s5(const TensorNHWC& x, const FilterKRSC& w, const Conv2DParams& p, TensorNHWCI32& y,
                            const S5* in_qp, const S5* f_qp) {
  regular(x, w, p, y, in_qp, f_qp);
}
void cpu_block_fprop_nhwc_qi32_u8(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p,
                                  TensorNHWCI32& y, const U8* in_qp, const U8* f_qp) {
  blocked(x, w, p, y, in_qp, f_qp);
}
void cpu_block_fprop_nhwc_qi32_s5(const TensorNHWC& x, const BlockFilterKByBxRSC& w, const BlockConv2DParams& p,
                                  TensorNHWCI32& y, const S5* in_qp, const S5* f_qp) {
  blocked(x, w, p, y, in_qp, f_qp);
}

}  // namespace conv_quant_detail
