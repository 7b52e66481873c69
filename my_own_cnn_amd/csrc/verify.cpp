// verify_tensors: element-wise absolute / relative comparison.  An element fails when its
// absolute error exceeds abs_eps and, where the reference value is not ~0, its relative
// error also exceeds rel_eps (the pass rule of /root/reference/src/verify.cpp:7-36).
// With abs_eps = rel_eps = 0 this is an exact check; int32 and int8 results compare
// exactly through float while their magnitude is below 2^24.

#include <algorithm>
#include <cmath>
#include <stdexcept>

#include "conv_types.h"

VerifyResult verify_tensors(const std::vector<float>& ref, const std::vector<float>& got, float abs_eps,
                            float rel_eps) {
  if (ref.size() != got.size()) throw std::runtime_error("verify_tensors size mismatch");
  VerifyResult res;
  bool all_ok = true;
  for (size_t i = 0; i < ref.size(); ++i) {
    const float mag = std::fabs(ref[i]);
    const float abs_err = std::fabs(ref[i] - got[i]);
    const float rel_err = abs_err / std::max(mag, 1e-6f);
    if (abs_err > res.max_abs_err) {
      res.max_abs_err = abs_err;
      res.max_abs_idx = i;
    }
    if (rel_err > res.max_rel_err) {
      res.max_rel_err = rel_err;
      res.max_rel_idx = i;
    }
    const bool rel_applies = mag > 1e-6f;
    if (abs_err > abs_eps && (!rel_applies || rel_err > rel_eps)) all_ok = false;
  }
  res.passed = all_ok;
  return res;
}
