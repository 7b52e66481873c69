"""The pointwise kernel (algo 'pointwise': 1x1 convolutions as a GEMM over the flattened pixels,
input streamed into LDS by loader waves) against the CPU oracle: every output byte bit-exact,
with and without ReLU and bias, on shapes that exercise its planner (one or two 64-channel tiles
per workgroup, 64 or 128 input channels, a last segment partly past the pixels, ranges of one
segment or of many, more workgroups than CUs), and the full ResNet-50 1x1 layer (C3) against the
accumulators the golden SHA-256 pins."""
import hashlib

import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W
from tests.golden import cases

pytestmark = pytest.mark.gpu

# (n, h, w, c, k)
SHAPES = [
    (1, 4, 4, 64, 64),       # one segment, one tile
    (2, 7, 7, 128, 128),     # 98 pixels: a partial last segment
    (3, 5, 9, 64, 192),      # k % 128 != 0: one tile per workgroup
    (1, 1, 1, 128, 64),      # a single pixel
    (2, 13, 11, 128, 256),
    (5, 3, 7, 64, 128),
    (8, 56, 56, 64, 256),    # 1568 segments
    (2, 28, 28, 128, 512),
    (40, 28, 28, 128, 128),  # ranges larger than the loader's 22 segments in flight
]


def _id(s):
    return "n{}h{}w{}c{}k{}".format(*s)


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_pointwise_matches_oracle(device, shape):
    n, h, wd, c, k = shape
    seed = 8100 + SHAPES.index(shape) * 8
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * c, seed + 1, -127, 127).reshape(k, 1, 1, c)
    bias = W.fill_i32_uniform(k, seed + 2, -4096, 4096)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    M.plan(M.make_desc(x.shape, w.shape, algo="pointwise"))  # accepted
    acc = oracle.conv_i8_acc(x, w, (0, 0, 1, 1, 1, 1, 1))
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    for relu in (False, True):
        for b in (bd, None):
            print(f"pointwise {_id(shape)} relu={relu} bias={b is not None}", flush=True)
            q = M.qconv2d_nhwc_i8(xd, wd_, b, sd, relu=relu, in_scale=0.02, algo="pointwise")
            torch.cuda.synchronize()
            want = oracle.requant_i8(acc, None if b is None else bias, ws, 0.02, 1.0, relu)
            np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"relu={relu} bias={b is not None}")


def test_pointwise_full_size_c3(device):
    wl = W.WORKLOADS["r50_1x1"]
    g = cases.config_goldens()["r50_1x1"]
    inp = wl.inputs()
    xd, wd = (torch.from_numpy(inp[k]).to(device) for k in ("x", "w"))
    bd, sd = (torch.from_numpy(inp[k]).to(device) for k in ("bias", "w_scale"))
    M.plan(M.make_desc(inp["x"].shape, inp["w"].shape, algo="pointwise"))
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd, algo="band")
    torch.cuda.synchronize()
    acc_h = acc.cpu().numpy()
    assert hashlib.sha256(acc_h.tobytes()).hexdigest() == g["acc_sha256"]
    for relu in (wl.relu, not wl.relu):
        print(f"pointwise r50_1x1 full size relu={relu}", flush=True)
        q = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=relu, in_scale=wl.in_scale, out_scale=wl.out_scale,
                              algo="pointwise")
        torch.cuda.synchronize()
        want = oracle.requant_i8(acc_h, inp["bias"], inp["w_scale"], wl.in_scale, wl.out_scale, relu)
        np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"relu={relu}")
