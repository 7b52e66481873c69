// HIP error checking and event timing for host code
// (counterpart of /root/reference/src/cuda_utils.h:1-25 and cuda_utils.cpp:1-23).
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

// Throws std::runtime_error naming the failing statement and its location, as the
// reference's cuda_check does (cuda_utils.h:7-11).
inline void hip_check(hipError_t err, const char* stmt, const char* file, int line) {
  if (err != hipSuccess) {
    throw std::runtime_error(std::string("HIP error at ") + file + ":" + std::to_string(line) + " in " + stmt +
                             " -> " + hipGetErrorString(err));
  }
}

#define HIP_CHECK(stmt) hip_check((stmt), #stmt, __FILE__, __LINE__)

// Elapsed time between two events recorded on one stream (default: the null stream).
class HipEventTimer {
 public:
  explicit HipEventTimer(hipStream_t stream = nullptr);
  ~HipEventTimer();
  HipEventTimer(const HipEventTimer&) = delete;
  HipEventTimer& operator=(const HipEventTimer&) = delete;

  void start();
  float stop_ms();  // records the stop event, waits for it, returns milliseconds

 private:
  hipStream_t stream_ = nullptr;
  hipEvent_t start_ = nullptr;
  hipEvent_t stop_ = nullptr;
};
