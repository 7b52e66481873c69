// GPU checks of the benchmark harness (TEST INFRASTRUCTURE ONLY): HipEventTimer and
// benchmark_cuda_op driven by a one-thread spin kernel whose duration is set per call, so
// the sample that lands at each sorted index is known in advance, and benchmark_cuda_op
// timing a libmiq_qconv convolution.  Prints one result per line; tests/test_gpu_harness.py
// compares them with the semantics of the reference's benchmark_cuda_op
// (/root/reference/src/bench.cpp:8-45): `warmup` untimed calls, then `iters` calls each
// bracketed by events, median = sorted[iters / 2], p90 = sorted[(size_t)(0.9f * (iters - 1))],
// gflops = flops / (median_ms * 1e6), std::runtime_error on warmup < 0 or iters <= 0.

#include <cstdio>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "conv_types.h"
#include "hip_utils.h"
#include "miq_qconv.h"

namespace {

// Spins one thread until the 100 MHz constant clock has advanced `ticks` (10 ns each); the
// loop also stops after `ticks * 64 + 4096` polls, so every launch ends.
__global__ void spin_kernel(long long ticks) {
  const long long t0 = __builtin_amdgcn_s_memrealtime();
  const long long cap = ticks * 64 + 4096;
  for (long long i = 0; i < cap; ++i) {
    if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

void spin_us(int us) {
  hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(1), 0, nullptr, static_cast<long long>(us) * 100);
  HIP_CHECK(hipGetLastError());
}

// benchmark_cuda_op over calls whose spin lengths (us) are `durations` in call order,
// after `warmup` calls of 50 us; prints the call count, median, p90 and gflops.
void programmed(const char* name, int warmup, const std::vector<int>& durations, size_t flops) {
  int calls = 0;
  const int iters = static_cast<int>(durations.size());
  const BenchResult r = benchmark_cuda_op(name, warmup, iters, flops, [&] {
    const int i = calls++;
    spin_us(i < warmup ? 50 : durations[static_cast<size_t>(i - warmup)]);
  });
  std::printf("programmed %s calls %d median_ms %.6f p90_ms %.6f gflops %.6g\n", name, calls, r.median_ms, r.p90_ms,
              r.gflops);
}

}  // namespace

int main() {
  // the event timer around one spin of known length
  {
    HipEventTimer t;
    spin_us(20);  // loads the kernel
    HIP_CHECK(hipDeviceSynchronize());
    for (int us : {200, 1000}) {
      t.start();
      spin_us(us);
      std::printf("timer spin_us %d ms %.6f\n", us, t.stop_ms());
    }
  }
  // sample order differs from call order; each list's sorted values are 100, 200, ... us
  programmed("n11", 3, {700, 300, 1100, 100, 900, 500, 200, 1000, 400, 800, 600}, 1000000000ull);
  programmed("n10", 0, {400, 1000, 100, 700, 300, 900, 200, 600, 800, 500}, 0);
  programmed("n2", 1, {600, 200}, 1000);
  programmed("n1", 2, {300}, 3000000000ull);
  for (const auto& bad : {std::make_pair(-1, 5), std::make_pair(0, 0), std::make_pair(2, -3)}) {
    int calls = 0;
    try {
      benchmark_cuda_op("bad", bad.first, bad.second, 0, [&] { ++calls; });
      std::printf("invalid %d %d no_throw calls %d\n", bad.first, bad.second, calls);
    } catch (const std::runtime_error& e) {
      std::printf("invalid %d %d threw \"%s\" calls %d\n", bad.first, bad.second, e.what(), calls);
    }
  }
  // benchmark_cuda_op around one libmiq_qconv launch (the fused int8 convolution of a
  // ResNet-style 3x3 layer, N=4), as a conv_bench-style caller would time it
  {
    miq_qconv_desc d{};
    d.n = 4; d.h = 56; d.w = 56; d.c = 64; d.k = 64; d.r = 3; d.s = 3;
    d.conv = miq_conv2d_params{1, 1, 1, 1, 1, 1, 1};
    d.relu = 1; d.in_scale = 0.02f; d.out_scale = 1.0f; d.algo = MIQ_ALGO_AUTO;
    const size_t xb = size_t(4) * 56 * 56 * 64, wb = size_t(64) * 9 * 64;
    int8_t *x = nullptr, *w = nullptr, *y = nullptr;
    int32_t* bias = nullptr;
    float* ws = nullptr;
    HIP_CHECK(hipMalloc(&x, xb));
    HIP_CHECK(hipMalloc(&w, wb));
    HIP_CHECK(hipMalloc(&y, xb));
    HIP_CHECK(hipMalloc(&bias, 64 * sizeof(int32_t)));
    HIP_CHECK(hipMalloc(&ws, 64 * sizeof(float)));
    HIP_CHECK(hipMemset(x, 1, xb));
    HIP_CHECK(hipMemset(w, 1, wb));
    HIP_CHECK(hipMemset(bias, 0, 64 * sizeof(int32_t)));
    std::vector<float> scale(64, 0.1f);
    HIP_CHECK(hipMemcpy(ws, scale.data(), 64 * sizeof(float), hipMemcpyHostToDevice));
    int status = MIQ_OK;
    int calls = 0;
    const size_t ops = size_t(2) * 4 * 56 * 56 * 64 * 9 * 64;
    const BenchResult r = benchmark_cuda_op("qconv", 5, 50, ops, [&] {
      ++calls;
      const int st = miq_qconv2d_nhwc_i8(&d, x, w, bias, ws, y, nullptr);
      if (st != MIQ_OK) status = st;
    });
    // pixel (0, 0) sees 4 of the 9 taps: relu(round(4 * 64 * 0.02 * 0.1)) = round(0.512) = 1
    int8_t y0 = -1;
    HIP_CHECK(hipMemcpy(&y0, y, 1, hipMemcpyDeviceToHost));
    std::printf("qconv status %d calls %d median_ms %.6f p90_ms %.6f gflops %.6g y0 %d\n", status, calls, r.median_ms,
                r.p90_ms, r.gflops, static_cast<int>(y0));
    HIP_CHECK(hipFree(x));
    HIP_CHECK(hipFree(w));
    HIP_CHECK(hipFree(y));
    HIP_CHECK(hipFree(bias));
    HIP_CHECK(hipFree(ws));
  }
  std::printf("done\n");
  return 0;
}
