// The reference's quant_conv_test (/root/reference/quant_conv_test.cu:14-228), re-expressed
// on HIP: the same four cases, generators and quantization parameters, calling the same
// C++ surface (cpu_fprop_nhwc_qi32<Tin>, launch_fprop_nhwc_qi32<Tin> and the blocked
// variants) and requiring exact int32 equality between the CPU path and this library.
// Also runs the int8 surface once through verify_tensors with exact tolerances.
// Exit code 0 and "quant_conv_test passed" on success.

#include <cstdint>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "conv_types.h"
#include "hip_utils.h"

namespace {

using nnalgebra::DataType;
template <DataType T>
using QParams = nnalgebra::QuantizationParameters<T>;

// Code generators of quant_conv_test.cu:17-35.
template <DataType T>
int code_at(size_t i, int salt);
template <>
int code_at<DataType::LinQuantU8>(size_t i, int salt) {
  return static_cast<int>((i * 37 + static_cast<size_t>(salt) * 19) % 251);
}
template <>
int code_at<DataType::LinQuantS5>(size_t i, int salt) {
  return static_cast<int>((i * 17 + static_cast<size_t>(salt) * 11) % 31) - 15;
}

template <DataType T>
void fill_codes(std::vector<float>& v, int salt) {
  for (size_t i = 0; i < v.size(); ++i) v[i] = static_cast<float>(code_at<T>(i, salt));
}

// Per-sample input parameters (quant_conv_test.cu:37-60) and filter parameters (:62-81).
template <DataType T>
std::vector<QParams<T>> sample_params(int n);
template <>
std::vector<QParams<DataType::LinQuantU8>> sample_params(int n) {
  std::vector<QParams<DataType::LinQuantU8>> v(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) {
    v[static_cast<size_t>(i)].zero_point = static_cast<uint8_t>(37 + 29 * i);
    v[static_cast<size_t>(i)].scale = 0.25f + 0.1f * static_cast<float>(i);
    v[static_cast<size_t>(i)].symmetric = false;
  }
  return v;
}
template <>
std::vector<QParams<DataType::LinQuantS5>> sample_params(int n) {
  std::vector<QParams<DataType::LinQuantS5>> v(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) {
    v[static_cast<size_t>(i)].zero_point = static_cast<int8_t>(-5 + 7 * i);
    v[static_cast<size_t>(i)].n_bins = 31;
    v[static_cast<size_t>(i)].scale = 0.5f + 0.125f * static_cast<float>(i);
  }
  return v;
}

template <DataType T>
QParams<T> filter_params();
template <>
QParams<DataType::LinQuantU8> filter_params() {
  QParams<DataType::LinQuantU8> q;
  q.zero_point = 91;
  q.scale = 0.75f;
  q.symmetric = false;
  return q;
}
template <>
QParams<DataType::LinQuantS5> filter_params() {
  QParams<DataType::LinQuantS5> q;
  q.zero_point = 3;
  q.n_bins = 31;
  q.scale = 0.875f;
  return q;
}

// Owning device allocation.
template <typename T>
class DeviceArray {
 public:
  explicit DeviceArray(size_t count) : count_(count) {
    if (count_ > 0) HIP_CHECK(hipMalloc(&ptr_, count_ * sizeof(T)));
  }
  ~DeviceArray() { (void)hipFree(ptr_); }
  DeviceArray(const DeviceArray&) = delete;
  DeviceArray& operator=(const DeviceArray&) = delete;
  T* get() { return ptr_; }
  void upload(const T* src) { HIP_CHECK(hipMemcpy(ptr_, src, count_ * sizeof(T), hipMemcpyHostToDevice)); }
  std::vector<T> download() const {
    std::vector<T> out(count_);
    HIP_CHECK(hipMemcpy(out.data(), ptr_, count_ * sizeof(T), hipMemcpyDeviceToHost));
    return out;
  }

 private:
  T* ptr_ = nullptr;
  size_t count_;
};

void require_equal(const std::vector<int32_t>& want, const std::vector<int32_t>& got, const std::string& label) {
  if (want.size() != got.size()) throw std::runtime_error(label + ": size mismatch");
  for (size_t i = 0; i < want.size(); ++i) {
    if (want[i] != got[i]) {
      std::ostringstream os;
      os << label << ": mismatch at " << i << " ref=" << want[i] << " got=" << got[i];
      throw std::runtime_error(os.str());
    }
  }
}

template <DataType T>
void regular_case(const std::string& label) {
  Conv2DParams p;
  p.pad_h = 1;
  p.pad_w = 0;
  p.stride_h = 1;
  p.stride_w = 1;
  p.dilation_h = 1;
  p.dilation_w = 1;
  p.groups = 2;
  TensorNHWC x(2, 5, 6, 4);
  FilterKRSC w(3, 2, x.c / p.groups, 6);
  fill_codes<T>(x.data, 1);
  fill_codes<T>(w.data, 7);
  const auto in_qp = sample_params<T>(x.n);
  const auto f_qp = filter_params<T>();

  TensorNHWCI32 y_cpu;
  cpu_fprop_nhwc_qi32<T>(x, w, p, y_cpu, in_qp.data(), &f_qp);

  DeviceArray<float> d_x(x.elements()), d_w(w.elements());
  DeviceArray<int32_t> d_y(y_cpu.elements());
  DeviceArray<QParams<T>> d_in(in_qp.size()), d_f(1);
  d_x.upload(x.ptr());
  d_w.upload(w.ptr());
  d_in.upload(in_qp.data());
  d_f.upload(&f_qp);
  launch_fprop_nhwc_qi32<T>(d_x.get(), d_w.get(), d_y.get(), x.n, x.h, x.w, x.c, w.r, w.s, w.k, p, d_in.get(),
                            d_f.get());
  HIP_CHECK(hipDeviceSynchronize());
  require_equal(y_cpu.data, d_y.download(), label);
}

template <DataType T>
void blocked_case(const std::string& label) {
  BlockConv2DParams p;
  p.conv.pad_h = 1;
  p.conv.pad_w = 1;
  p.conv.stride_h = 1;
  p.conv.stride_w = 1;
  p.conv.dilation_h = 1;
  p.conv.dilation_w = 1;
  p.conv.groups = 1;
  p.block_by = 2;
  p.block_bx = 3;
  TensorNHWC x(2, 6, 6, 4);
  BlockFilterKByBxRSC w(5, p.block_by, p.block_bx, 3, 3, x.c / p.conv.groups);
  fill_codes<T>(x.data, 3);
  fill_codes<T>(w.data, 9);
  const auto in_qp = sample_params<T>(x.n);
  const auto f_qp = filter_params<T>();

  TensorNHWCI32 y_cpu;
  cpu_block_fprop_nhwc_qi32<T>(x, w, p, y_cpu, in_qp.data(), &f_qp);

  DeviceArray<float> d_x(x.elements()), d_w(w.elements());
  DeviceArray<int32_t> d_y(y_cpu.elements());
  DeviceArray<QParams<T>> d_in(in_qp.size()), d_f(1);
  d_x.upload(x.ptr());
  d_w.upload(w.ptr());
  d_in.upload(in_qp.data());
  d_f.upload(&f_qp);
  launch_block_fprop_nhwc_qi32<T>(d_x.get(), d_w.get(), d_y.get(), x.n, x.h, x.w, x.c, w.r, w.s, w.k, p, d_in.get(),
                                  d_f.get());
  HIP_CHECK(hipDeviceSynchronize());
  require_equal(y_cpu.data, d_y.download(), label);
}

// The int8 surface: accumulators against the S5 CPU path with zero points 0, compared
// through verify_tensors with zero tolerances.
void int8_case() {
  Conv2DParams p;  // 3x3, stride 1, pad 1
  const int n = 2, h = 9, w = 11, c = 32, k = 48;
  TensorNHWC x(n, h, w, c);
  FilterKRSC f(3, 3, c, k);
  std::vector<int8_t> x8(x.elements()), f8(f.elements());
  for (size_t i = 0; i < x8.size(); ++i) {
    x8[i] = static_cast<int8_t>(static_cast<int>((i * 2654435761u) >> 7 & 0xff) - 128);
    x.data[i] = x8[i];
  }
  for (size_t i = 0; i < f8.size(); ++i) {
    f8[i] = static_cast<int8_t>(static_cast<int>((i * 40503u + 17u) >> 3 & 0xff) - 128);
    f.data[i] = f8[i];
  }
  std::vector<QParams<DataType::LinQuantS5>> zq(static_cast<size_t>(n));
  QParams<DataType::LinQuantS5> fq;
  TensorNHWCI32 y_cpu;
  cpu_fprop_nhwc_qi32<DataType::LinQuantS5>(x, f, p, y_cpu, zq.data(), &fq);

  DeviceArray<int8_t> d_x(x8.size()), d_f(f8.size());
  DeviceArray<int32_t> d_y(y_cpu.elements());
  d_x.upload(x8.data());
  d_f.upload(f8.data());
  launch_fprop_nhwc_qi8_acc32(d_x.get(), d_f.get(), d_y.get(), n, h, w, c, 3, 3, k, p);
  HIP_CHECK(hipDeviceSynchronize());
  const auto got = d_y.download();
  const std::vector<float> a(y_cpu.data.begin(), y_cpu.data.end()), b(got.begin(), got.end());
  const VerifyResult v = verify_tensors(a, b, 0.0f, 0.0f);
  if (!v.passed) {
    std::ostringstream os;
    os << "int8_acc32: max_abs_err " << v.max_abs_err << " at " << v.max_abs_idx;
    throw std::runtime_error(os.str());
  }
}

}  // namespace

int main() {
  try {
    regular_case<DataType::LinQuantU8>("regular_u8");
    regular_case<DataType::LinQuantS5>("regular_s5");
    blocked_case<DataType::LinQuantU8>("blocked_u8");
    blocked_case<DataType::LinQuantS5>("blocked_s5");
    int8_case();
    std::cout << "quant_conv_test passed\n";
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "quant_conv_test failed: " << e.what() << "\n";
    return 1;
  }
}
