"""Hardware facts the kernels are designed around, measured by tests/hw/bin/hw_probes on the
GPU: the launch floor in a HIP graph, per-CU global->LDS ingest (L2 faster than HBM), the
ds_read_b128 lane-to-cycle rule for bank conflicts, and MFMA issue rates.  Margins are wide:
these pin the shape of each fact (which rule predicts the LDS timings, which source is faster,
where the floors lie), not exact rates that vary from box to box."""
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "hw" / "bin" / "hw_probes"


def _run(what, device, timeout):
    assert EXE.exists(), f"{EXE} is missing: build with __graft_entry__.build()"
    print(f"hw_probes {what}", flush=True)
    out = subprocess.run([str(EXE), what], capture_output=True, text=True, timeout=timeout)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.rstrip().endswith("done")
    return out.stdout


def test_launch_floor_in_a_graph(device):
    rows = re.findall(r"launch grid (\d+) block (\d+) eager_us ([\d.]+) graph_us ([\d.]+)", _run("launch", device, 60))
    assert len(rows) == 6
    for grid, block, eager, graph in rows:
        # an empty kernel back to back in a graph: about 1.5 us per launch, never near the
        # tens of microseconds of the convolutions themselves
        assert 0.3 < float(graph) < 3.0, (grid, block, graph)
        assert float(eager) < 10.0


def test_lds_bank_rule(device):
    out = _run("lds", device, 90)
    rates = re.findall(r"lds_rate waves (\d+) us [\d.]+ bytes_per_clk_per_cu ([\d.]+)", out)
    assert len(rates) == 5
    rate = {int(w): float(b) for w, b in rates}
    assert rate[8] > 2.5 * rate[1]  # one wave cannot keep the LDS busy; eight nearly can
    pats = re.findall(r"lds_pattern (\S+) rel_time ([\d.]+) parity_rule (\d+) consecutive_rule (\d+)", out)
    assert len(pats) >= 200
    rel = np.array([float(p[1]) for p in pats])
    par = np.array([int(p[2]) for p in pats]) / 4.0
    con = np.array([int(p[3]) for p in pats]) / 4.0

    def worst_misfit(pred):
        # time = a + b * predicted cycles, least squares; the largest relative residual
        a, b = np.polyfit(pred, rel, 1)[::-1]
        return float(np.max(np.abs(rel - (a + b * pred)) / rel)), b

    par_err, par_slope = worst_misfit(par)
    con_err, _ = worst_misfit(con)
    print(f"parity rule worst misfit {par_err:.3f} (slope {par_slope:.3f}); consecutive rule {con_err:.3f}")
    assert par_slope > 0.5  # conflicts cost time in proportion to the extra cycles
    assert par_err < 0.12
    assert par_err < con_err
    named = {p[0]: (float(p[1]), int(p[2])) for p in pats}
    # lanes l and l + 16 read one slot class without conflict; a broadcast costs nothing extra
    assert named["l_and_l16_same_class"][1] == 4 and named["l_and_l16_same_class"][0] < 1.1
    assert named["broadcast"][0] < 1.1


def test_ingest_l2_faster_than_hbm(device):
    rows = re.findall(r"ingest source (\w+) kb (\d+) waves (\d+) wg_us ([\d.]+) gbs_per_cu ([\d.]+)",
                      _run("ingest", device, 90))
    assert len(rows) == 16
    gbs = {(src, int(kb), int(w)): float(g) for src, kb, w, _, g in rows}
    for kb in (36, 72, 144):
        assert gbs[("l2", kb, 8)] > gbs[("hbm", kb, 8)]
    # per-CU ingest grows with the bytes in flight and stays far below the 8 TB/s / 256 CUs
    # of HBM spread evenly (31 GB/s per CU) only for small loads
    assert gbs[("l2", 144, 8)] > gbs[("l2", 8, 8)]


def test_mfma_issue_rates(device):
    rows = re.findall(r"mfma shape (\d+)x\d+ chains (\d+) valu (\d+) ds_read (\d+) waves_per_simd (\d+) "
                      r"ns_per_mfma ([\d.]+) tops ([\d.]+) peak_frac ([\d.]+)", _run("mfma", device, 90))
    assert len(rows) == 17
    frac = {tuple(int(v) for v in r[:5]): float(r[7]) for r in rows}
    # enough independent chains reach most of the dense int8 peak
    assert frac[(16, 8, 0, 0, 1)] > 0.75 and frac[(32, 4, 0, 0, 1)] > 0.8
    # 16 VALU ops per MFMA group of one wave halve the MFMA rate; a second wave per SIMD hides 8
    assert frac[(16, 4, 16, 0, 1)] < 0.7 * frac[(16, 4, 0, 0, 1)]
    assert frac[(16, 4, 8, 0, 2)] > frac[(16, 4, 8, 0, 1)]
