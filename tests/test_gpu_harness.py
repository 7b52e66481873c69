"""The C++ benchmark harness on the GPU: HipEventTimer and benchmark_cuda_op
(my_own_cnn_amd/csrc/bench.cpp) against the semantics of the reference's benchmark_cuda_op
(/root/reference/src/bench.cpp:8-45).

tests/cpp/bin/bench_harness_gpu times a spin kernel whose length is set per call, in an
order that differs from the sorted order, so each reported statistic names the sorted index
it was taken from: median = sorted[n // 2] (the upper middle for even n, not a mean),
p90 = sorted[int(float32(0.9) * float32(n - 1))], gflops = flops / (median_ms * 1e6); the
warmup calls are made and not timed; warmup < 0 or iters <= 0 throws before any call."""
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "bin" / "bench_harness_gpu"

# name -> (warmup, spin lengths in us in call order, flops); as in bench_harness_gpu.cpp
PROGRAMMED = {
    "n11": (3, [700, 300, 1100, 100, 900, 500, 200, 1000, 400, 800, 600], 1000000000),
    "n10": (0, [400, 1000, 100, 700, 300, 900, 200, 600, 800, 500], 0),
    "n2": (1, [600, 200], 1000),
    "n1": (2, [300], 3000000000),
}


def reference_stats(durations_us):
    """Median and p90 sample (ms) under the reference's index rule, float32 arithmetic."""
    s = sorted(durations_us)
    n = len(s)
    p90_idx = int(np.float32(0.9) * np.float32(n - 1))
    return s[n // 2] / 1e3, s[p90_idx] / 1e3


@pytest.fixture(scope="module")
def harness_output(device):
    assert EXE.exists(), f"{EXE} is missing: build with __graft_entry__.build()"
    print("bench_harness_gpu", flush=True)
    out = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=100)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.rstrip().endswith("done")
    return out.stdout


def _close(measured_ms, want_ms):
    # a spin of t us measures t us plus launch latency (a few us) and clock granularity
    return want_ms - 0.005 <= measured_ms <= want_ms * 1.05 + 0.03


def test_event_timer_measures_a_known_spin(harness_output):
    rows = re.findall(r"timer spin_us (\d+) ms ([\d.]+)", harness_output)
    assert len(rows) == 2
    for us, ms in rows:
        assert _close(float(ms), int(us) / 1e3), (us, ms)


@pytest.mark.parametrize("name", sorted(PROGRAMMED))
def test_benchmark_cuda_op_statistics(harness_output, name):
    warmup, durations, flops = PROGRAMMED[name]
    m = re.search(rf"programmed {name} calls (\d+) median_ms ([\d.]+) p90_ms ([\d.]+) gflops (\S+)", harness_output)
    assert m, harness_output
    calls, med, p90, gflops = int(m[1]), float(m[2]), float(m[3]), float(m[4])
    assert calls == warmup + len(durations)  # every warmup call made, none of them timed
    want_med, want_p90 = reference_stats(durations)
    assert _close(med, want_med), (name, med, want_med)
    assert _close(p90, want_p90), (name, p90, want_p90)
    # the spins are 100 us apart: each statistic identifies exactly one sorted index
    assert abs(med - want_med) < 0.05 and abs(p90 - want_p90) < 0.05
    want_gflops = flops / (med * 1e6) if med > 0 else 0.0
    assert gflops == pytest.approx(want_gflops, rel=1e-4, abs=1e-6)


def test_even_count_median_is_the_upper_middle_and_p90_can_be_below_it(harness_output):
    # n = 2: the reference takes sorted[1] as the median and sorted[int(0.9f * 1)] = sorted[0]
    # as p90, so p90 < median; a harness that averaged or rounded up would not
    m = re.search(r"programmed n2 calls \d+ median_ms ([\d.]+) p90_ms ([\d.]+)", harness_output)
    med, p90 = float(m[1]), float(m[2])
    assert med > 0.5 and p90 < 0.3 and p90 < med


def test_invalid_counts_throw_before_any_call(harness_output):
    rows = re.findall(r"invalid (-?\d+) (-?\d+) (\S+) (.*) calls (\d+)", harness_output)
    assert len(rows) == 3
    for warm, iters, what, msg, calls in rows:
        assert what == "threw", (warm, iters)
        assert "invalid benchmark warmup/iters" in msg
        assert int(calls) == 0


def test_benchmark_cuda_op_times_a_library_convolution(harness_output):
    m = re.search(r"qconv status (\d+) calls (\d+) median_ms ([\d.]+) p90_ms ([\d.]+) gflops (\S+) y0 (-?\d+)",
                  harness_output)
    assert m, harness_output
    status, calls, med, p90, gflops, y0 = int(m[1]), int(m[2]), float(m[3]), float(m[4]), float(m[5]), int(m[6])
    assert status == 0 and calls == 55 and y0 == 1
    # 4 x 56 x 56 x 64 x 64 x 9 MACs: per-launch event pairs see it in well under a millisecond
    assert 0 < med <= p90 < 1.0
    assert gflops == pytest.approx(2 * 4 * 56 * 56 * 64 * 9 * 64 / (med * 1e6), rel=1e-4)
