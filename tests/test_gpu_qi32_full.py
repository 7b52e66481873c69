"""The float-code convolution (launch_fprop_nhwc_qi32, the reference's own API) at the full C2,
C4 and C5 sizes against the sha256 of the reference's cpu_fprop_nhwc_qi32 on the same inputs
(tests/golden/qi32_full.json, written from oracle/_ref): AUTO (the row-band kernel on C2, the
stream route on C4, the stem route on C5), the caller-workspace entry point miq_fprop_nhwc_qi32_ws, and that entry
point recorded into a HIP graph and replayed, with eager work and synchronisations between
replays and no device memory allocated by the captured call."""
import hashlib

import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
from tests.golden import cases
from tests.test_gpu_parity import dev, qparams_dev

pytestmark = pytest.mark.gpu

PLAN = {"c2_u8": "band", "c2_s5": "band", "c4_u8": "stream", "c5_u8": "stem_s2d"}


def _problem(name, device):
    kind, x, w, conv, zp, fzp = cases.qi32_full_inputs(name)
    n, h, wd, c = x.shape
    k, r, s = w.shape[0], w.shape[1], w.shape[2]
    tin, in_qp = qparams_dev(kind, zp, device)
    _, f_qp = qparams_dev(kind, [fzp], device)
    p = M.Conv2DParams(*conv)
    ho, wo = M.infer_conv_shape(n, h, wd, c, r, s, k, p)
    return dict(tin=tin, x=dev(x, device), w=dev(w, device), in_qp=in_qp, f_qp=f_qp, p=p,
                dims=(n, h, wd, c, r, s, k), yshape=(n, ho, wo, k))


def _sha(y):
    return hashlib.sha256(y.cpu().numpy().tobytes()).hexdigest()


def _run(pr, y, **kw):
    n, h, wd, c, r, s, k = pr["dims"]
    M.fprop_nhwc_qi32_algo(pr["tin"], pr["x"], pr["w"], y, n, h, wd, c, r, s, k, pr["p"], pr["in_qp"], pr["f_qp"],
                           **kw)


@pytest.mark.parametrize("name", list(cases.QI32_FULL))
def test_qi32_full_size_matches_reference_sha(device, name):
    g = cases.qi32_full_goldens()[name]
    pr = _problem(name, device)
    n, h, wd, c, r, s, k = pr["dims"]
    assert M.plan_qi32(n, h, wd, c, r, s, k, pr["p"]) == PLAN[name]
    print(f"qi32 full {name}: AUTO", flush=True)
    y = torch.full(pr["yshape"], -7, dtype=torch.int32, device=device)
    M.launch_fprop_nhwc_qi32(pr["tin"], pr["x"], pr["w"], y, n, h, wd, c, r, s, k, pr["p"], pr["in_qp"], pr["f_qp"])
    torch.cuda.synchronize()
    assert _sha(y) == g["sha256"]
    print(f"qi32 full {name}: caller workspace", flush=True)
    need = M.qi32_workspace_size(n, h, wd, c, r, s, k, pr["p"])
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    y2 = torch.full(pr["yshape"], 5, dtype=torch.int32, device=device)
    _run(pr, y2, workspace=ws, workspace_bytes=need)
    torch.cuda.synchronize()
    assert _sha(y2) == g["sha256"]


@pytest.mark.parametrize("name", ["c2_u8", "c4_u8", "c5_u8"])
def test_qi32_ws_in_a_graph(device, name):
    g = cases.qi32_full_goldens()[name]
    pr = _problem(name, device)
    n, h, wd, c, r, s, k = pr["dims"]
    need = M.qi32_workspace_size(n, h, wd, c, r, s, k, pr["p"])
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    y = torch.full(pr["yshape"], -7, dtype=torch.int32, device=device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    graph = torch.cuda.CUDAGraph()
    print(f"qi32 graph {name}: capture", flush=True)
    with torch.cuda.graph(graph, stream=side):
        _run(pr, y, workspace=ws, workspace_bytes=need, stream=side)
    torch.cuda.synchronize()
    for rep in range(3):
        y.fill_(rep - 9)                 # eager work between replays
        torch.cuda.synchronize()
        print(f"qi32 graph {name}: replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert _sha(y) == g["sha256"], f"replay {rep}"
    free1 = torch.cuda.mem_get_info()[0]
    # nothing of the workspace's size was allocated by the captured call or its replays
    assert free0 - free1 < max(need // 2, 4 << 20), (free0, free1, need)
