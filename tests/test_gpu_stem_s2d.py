"""The space-to-depth stem kernel (algo 'stem_s2d': stride-2 thin-channel convolutions as a
stride-1 convolution over 2 x 2 x c pixels built in LDS) against the CPU oracle: every output
byte bit-exact, with and without ReLU and bias, on filters of 1x1 to 7x7 (odd and even, square
and not), 1 to 4 channels, padding 0..3 (also unequal), a partly empty last segment of a row,
bands cut short, and the full ResNet-50 stem (C5) against the accumulators its golden SHA-256
pins."""
import hashlib

import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W
from tests.golden import cases

pytestmark = pytest.mark.gpu

# (n, h, w, c, k, r, s, ph, pw)
SHAPES = [
    (2, 20, 16, 3, 64, 7, 7, 3, 3),
    (2, 21, 48, 3, 64, 7, 7, 3, 3),     # Wo = 24: a partly empty segment
    (1, 9, 16, 1, 64, 3, 3, 1, 1),
    (2, 13, 8, 2, 128, 5, 5, 2, 2),     # two 64-channel tiles
    (1, 10, 4, 4, 64, 4, 4, 1, 1),      # even filter, c = 4 (16-byte s2d pixels full)
    (3, 7, 32, 3, 64, 1, 1, 0, 0),      # 1x1 stride 2
    (2, 11, 48, 3, 64, 7, 7, 0, 0),     # no padding
    (1, 9, 16, 3, 64, 3, 2, 1, 0),      # unequal filter and padding
    (1, 224, 224, 3, 64, 7, 7, 3, 3),   # one full stem image
    (5, 33, 16, 3, 64, 7, 7, 3, 3),
    # the row build reads each pixel pair's 4C bytes from an offset (PLB - pw C) mod 4 into its
    # first dword: 1 and 2 for three channels, 2 for two and for one channel
    (2, 15, 32, 3, 64, 3, 3, 1, 1),
    (1, 12, 48, 3, 64, 5, 5, 2, 2),
    (2, 11, 24, 2, 64, 3, 3, 1, 1),
    (1, 10, 32, 1, 64, 5, 5, 2, 2),
]


def _id(s):
    return "n{}h{}w{}c{}k{}r{}s{}p{}{}".format(*s)


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_stem_s2d_matches_oracle(device, shape):
    n, h, wd, c, k, r, s, ph, pw = shape
    seed = 8700 + SHAPES.index(shape) * 8
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * c, seed + 1, -127, 127).reshape(k, r, s, c)
    bias = W.fill_i32_uniform(k, seed + 2, -4096, 4096)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(stride=2, padding=(ph, pw))
    M.plan(M.make_desc(x.shape, w.shape, algo="stem_s2d", **kw))  # accepted
    acc = oracle.conv_i8_acc(x, w, (ph, pw, 2, 2, 1, 1, 1))
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    for relu in (False, True):
        for b in (bd, None):
            print(f"stem_s2d {_id(shape)} relu={relu} bias={b is not None}", flush=True)
            q = M.qconv2d_nhwc_i8(xd, wd_, b, sd, relu=relu, in_scale=0.02, algo="stem_s2d", **kw)
            torch.cuda.synchronize()
            want = oracle.requant_i8(acc, None if b is None else bias, ws, 0.02, 1.0, relu)
            np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"relu={relu} bias={b is not None}")


def test_stem_s2d_full_size_c5(device):
    wl = W.WORKLOADS["stem"]
    g = cases.config_goldens()["stem"]
    inp = wl.inputs()
    xd, wd = (torch.from_numpy(inp[k]).to(device) for k in ("x", "w"))
    bd, sd = (torch.from_numpy(inp[k]).to(device) for k in ("bias", "w_scale"))
    kw = dict(stride=wl.stride, padding=wl.pad)
    assert M.plan(M.make_desc(inp["x"].shape, inp["w"].shape, **kw)) == "stem_s2d"  # AUTO's choice
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd, algo="stem", **kw)
    torch.cuda.synchronize()
    acc_h = acc.cpu().numpy()
    assert hashlib.sha256(acc_h.tobytes()).hexdigest() == g["acc_sha256"]
    for relu in (wl.relu, not wl.relu):
        print(f"stem_s2d stem full size relu={relu}", flush=True)
        q = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=relu, in_scale=wl.in_scale, out_scale=wl.out_scale,
                              algo="stem_s2d", **kw)
        torch.cuda.synchronize()
        want = oracle.requant_i8(acc_h, inp["bias"], inp["w_scale"], wl.in_scale, wl.out_scale, relu)
        np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"relu={relu}")
