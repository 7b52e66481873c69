"""The row-pipelined band kernel (algo 'pipe': input rows streamed into LDS by a loader wave,
per-row LDS flags) against the CPU oracle: every output byte bit-exact, with and without ReLU,
on shapes that exercise its planner and addressing (bands of 1..many rows, a last band cut
short, segments crossing row ends, the band's last segment partly empty, padding 0/1/2,
dilation, 1x1 and 3x3 filters, widths 8..96, no bias), and at the full ResNet-50 3x3 size
against the accumulators the golden SHA-256 pins."""
import hashlib

import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W
from tests.golden import cases

pytestmark = pytest.mark.gpu

# (n, h, w, r, s, pad, dilation)
SHAPES = [
    (1, 8, 8, 3, 3, 1, 1),
    (2, 56, 56, 3, 3, 1, 1),
    (1, 5, 16, 3, 3, 1, 1),
    (3, 13, 24, 3, 3, 1, 1),
    (1, 30, 40, 3, 3, 0, 1),   # Wo = 38: rejected (Wo % 8), AUTO takes another kernel
    (2, 17, 32, 3, 3, 2, 2),
    (1, 28, 64, 3, 3, 1, 1),
    (1, 9, 96, 3, 3, 1, 1),
    (2, 11, 40, 1, 1, 0, 1),
    (1, 3, 8, 1, 1, 0, 1),
    (4, 7, 56, 3, 3, 1, 1),
    (40, 16, 16, 3, 3, 1, 1),  # many images: bands of several rows
    (20, 30, 24, 3, 3, 1, 1),
]


def _id(s):
    return "n{}h{}w{}r{}s{}p{}d{}".format(*s)


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_pipe_matches_oracle(device, shape):
    n, h, wd, r, s, pad, dil = shape
    c = k = 64
    seed = 5100 + SHAPES.index(shape) * 8
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * c, seed + 1, -127, 127).reshape(k, r, s, c)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=pad, dilation=dil)
    conv = (pad, pad, 1, 1, dil, dil, 1)
    wo = wd + 2 * pad - dil * (s - 1)
    eligible = wo % 8 == 0
    try:
        M.plan(M.make_desc(x.shape, w.shape, algo="pipe", **kw))
        planned = True
    except M.MiqError:
        planned = False
    assert planned == eligible
    if not eligible:
        return
    acc = oracle.conv_i8_acc(x, w, conv)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    for relu in (False, True):
        for b in (bd, None):
            print(f"pipe {_id(shape)} relu={relu} bias={b is not None}", flush=True)
            q = M.qconv2d_nhwc_i8(xd, wd_, b, sd, relu=relu, in_scale=0.02, algo="pipe", **kw)
            torch.cuda.synchronize()
            want = oracle.requant_i8(acc, None if b is None else bias, ws, 0.02, 1.0, relu)
            np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"relu={relu} bias={b is not None}")


def test_pipe_full_size_headline(device):
    wl = W.WORKLOADS["r50_3x3"]
    g = cases.config_goldens()["r50_3x3"]
    inp = wl.inputs()
    xd, wd = (torch.from_numpy(inp[k]).to(device) for k in ("x", "w"))
    bd, sd = (torch.from_numpy(inp[k]).to(device) for k in ("bias", "w_scale"))
    kw = dict(stride=wl.stride, padding=wl.pad)
    M.plan(M.make_desc(inp["x"].shape, inp["w"].shape, algo="pipe", **kw))  # accepted
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd, algo="band", **kw)
    torch.cuda.synchronize()
    acc_h = acc.cpu().numpy()
    assert hashlib.sha256(acc_h.tobytes()).hexdigest() == g["acc_sha256"]
    for relu in (wl.relu, not wl.relu):
        print(f"pipe r50_3x3 full size relu={relu}", flush=True)
        q = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=relu, in_scale=wl.in_scale, out_scale=wl.out_scale, algo="pipe",
                              **kw)
        torch.cuda.synchronize()
        want = oracle.requant_i8(acc_h, inp["bias"], inp["w_scale"], wl.in_scale, wl.out_scale, relu)
        np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"relu={relu}")


def test_pipe_rejects_other_outputs(device):
    x = torch.zeros((1, 8, 8, 64), dtype=torch.int8, device=device)
    w = torch.zeros((64, 3, 3, 64), dtype=torch.int8, device=device)
    with pytest.raises(M.MiqError):
        M.qconv2d_nhwc_i8_acc32(x, w, padding=1, algo="pipe")
