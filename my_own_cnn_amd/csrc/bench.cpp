// HIP event timing and the benchmark loop of the harness
// (counterparts of /root/reference/src/cuda_utils.cpp:1-23 and src/bench.cpp:8-45).

#include <algorithm>
#include <stdexcept>
#include <vector>

#include "conv_types.h"
#include "hip_utils.h"

HipEventTimer::HipEventTimer(hipStream_t stream) : stream_(stream) {
  HIP_CHECK(hipEventCreate(&start_));
  HIP_CHECK(hipEventCreate(&stop_));
}

HipEventTimer::~HipEventTimer() {
  (void)hipEventDestroy(start_);
  (void)hipEventDestroy(stop_);
}

void HipEventTimer::start() { HIP_CHECK(hipEventRecord(start_, stream_)); }

float HipEventTimer::stop_ms() {
  HIP_CHECK(hipEventRecord(stop_, stream_));
  HIP_CHECK(hipEventSynchronize(stop_));
  float ms = 0.0f;
  HIP_CHECK(hipEventElapsedTime(&ms, start_, stop_));
  return ms;
}

// `warmup` untimed calls, then `iters` calls each bracketed by events on the null stream;
// reports the median and the 90th-percentile sample (index floor(0.9*(iters-1))) and the
// GFLOP/s of the median.
BenchResult benchmark_cuda_op(const std::string& op_name, int warmup, int iters, size_t flops,
                              const std::function<void()>& fn) {
  (void)op_name;
  if (warmup < 0 || iters <= 0) throw std::runtime_error("invalid benchmark warmup/iters");
  for (int i = 0; i < warmup; ++i) fn();
  HIP_CHECK(hipDeviceSynchronize());

  std::vector<float> ms(static_cast<size_t>(iters));
  HipEventTimer timer;
  for (int i = 0; i < iters; ++i) {
    timer.start();
    fn();
    ms[static_cast<size_t>(i)] = timer.stop_ms();
  }
  std::sort(ms.begin(), ms.end());
  BenchResult out;
  out.median_ms = ms[ms.size() / 2];
  out.p90_ms = ms[static_cast<size_t>(0.9f * static_cast<float>(ms.size() - 1))];
  out.gflops = out.median_ms > 0.0f
                   ? static_cast<float>(static_cast<double>(flops) / (static_cast<double>(out.median_ms) * 1.0e6))
                   : 0.0f;
  return out;
}
