// CPU-only checks of the C++ surface that need no GPU: verify_tensors on crafted vectors
// (printed one result per line for the Python test to compare with the reference's
// verify_tensors), and the shape-inference exceptions of the drop-in headers.

#include <cmath>
#include <cstdio>
#include <limits>
#include <stdexcept>
#include <vector>

#include "conv_types.h"

namespace {

void emit(const char* name, const std::vector<float>& a, const std::vector<float>& b, float ae, float re) {
  const VerifyResult v = verify_tensors(a, b, ae, re);
  std::printf("%s %.9g %.9g %zu %zu %d\n", name, v.max_abs_err, v.max_rel_err, v.max_abs_idx, v.max_rel_idx,
              v.passed ? 1 : 0);
}

}  // namespace

int main() {
  emit("exact_equal", {1.f, -2.f, 3.5f}, {1.f, -2.f, 3.5f}, 0.f, 0.f);
  emit("one_off", {100.f, 200.f, 300.f}, {100.f, 201.f, 300.f}, 0.f, 0.f);
  emit("within_abs", {1.f, 2.f}, {1.00005f, 2.f}, 1e-4f, 0.f);
  emit("within_rel", {1000.f, 2.f}, {1000.5f, 2.f}, 1e-4f, 1e-3f);
  emit("zero_ref", {0.f, 0.f}, {1e-7f, 3e-3f}, 1e-4f, 1e-3f);
  emit("tiny_ref", {1e-7f, 5.f}, {2e-7f, 5.f}, 0.f, 0.f);
  emit("negative", {-4.f, -8.f}, {-4.004f, -8.f}, 1e-4f, 1e-3f);
  emit("empty", {}, {}, 0.f, 0.f);
  bool threw = false;
  try {
    verify_tensors({1.f}, {1.f, 2.f}, 0.f, 0.f);
  } catch (const std::runtime_error&) {
    threw = true;
  }
  std::printf("size_mismatch_throws %d\n", threw ? 1 : 0);

  // shape inference messages of the drop-in header
  const struct {
    int c, k, groups, h, pad, r, stride;
  } bad[] = {{4, 4, 0, 5, 1, 3, 1}, {4, 4, 3, 5, 1, 3, 1}, {6, 4, 3, 5, 1, 3, 1}, {4, 4, 1, 2, 0, 5, 1}, {4, 4, 1, 5, 1, 3, 0}};
  for (const auto& b : bad) {
    Conv2DParams p;
    p.groups = b.groups;
    p.pad_h = p.pad_w = b.pad;
    p.stride_h = p.stride_w = b.stride;
    TensorNHWC x(1, b.h, b.h, b.c);
    FilterKRSC w(b.r, b.r, b.groups > 0 ? b.c / b.groups : 0, b.k);
    try {
      infer_conv_shape(x, w, p);
      std::printf("shape ok\n");
    } catch (const std::runtime_error& e) {
      std::printf("shape error: %s\n", e.what());
    }
  }
  return 0;
}
