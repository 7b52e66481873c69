"""The vector-ALU int8 kernel (i8_dot4_kernel, MIQ_ALGO_DOT4: v_dot4_i32_i8, no matrix
instructions) against the oracle, bit for bit, on the shapes it exists for and its edges:
thin input channels (C = 1, 2, 3, 5 with the byte-packed gather), few output channels (K = 1
.. 40, every channel-tile width and partial tiles), 1x1 and 7x7 filters, stride, dilation,
padding, groups, and an output whose channel runs are not 4-byte aligned.  All three output
stages (int32 accumulators, requantized int8 with and without ReLU, fp32 view)."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W

pytestmark = pytest.mark.gpu

# n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups)
SHAPES = [
    (2, 30, 30, 3, 16, 7, 7, (3, 3, 2, 2, 1, 1, 1)),      # stem-like, C = 3
    (1, 17, 19, 1, 8, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    (2, 9, 11, 2, 4, 3, 5, (2, 1, 1, 2, 1, 1, 1)),
    (1, 12, 12, 5, 12, 3, 3, (1, 1, 1, 1, 2, 2, 1)),
    (2, 14, 14, 64, 1, 1, 1, (0, 0, 1, 1, 1, 1, 1)),      # 1x1, K = 1
    (2, 14, 14, 64, 3, 1, 1, (0, 0, 1, 1, 1, 1, 1)),
    (2, 14, 14, 64, 8, 1, 1, (0, 0, 1, 1, 1, 1, 1)),
    (2, 14, 14, 128, 16, 1, 1, (0, 0, 1, 1, 1, 1, 1)),
    (2, 14, 14, 64, 24, 1, 1, (0, 0, 2, 2, 1, 1, 1)),     # KT 32, partial tile
    (1, 10, 10, 32, 40, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # two tiles, the second partial
    (2, 11, 13, 32, 12, 3, 3, (1, 1, 1, 1, 1, 1, 4)),     # groups: 8 -> 3 per group
    (1, 8, 8, 12, 6, 3, 3, (1, 1, 1, 1, 1, 1, 3)),        # c/groups = 4, k/groups = 2
    (1, 9, 9, 6, 6, 3, 3, (1, 1, 1, 1, 1, 1, 6)),         # depthwise, byte gather
]


def _id(s):
    n, h, w, c, k, r, sz, conv = s
    return f"n{n}h{h}w{w}c{c}k{k}r{r}s{sz}s{conv[2]}d{conv[4]}g{conv[6]}"


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_dot4_bit_exact(device, shape):
    n, h, wd, c, k, r, s, conv = shape
    g = conv[6]
    seed = 4100 + SHAPES.index(shape) * 8
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * (c // g), seed + 1, -127, 127).reshape(k, r, s, c // g)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=g)
    assert M.plan(M.make_desc(x.shape, w.shape, algo="dot4", **kw)) == "dot4"
    acc_want = oracle.conv_i8_acc(x, w, conv)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd_, algo="dot4", **kw)
    q0 = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=False, in_scale=0.02, algo="dot4", **kw)
    q1 = M.qconv2d_nhwc_i8(xd, wd_, None, sd, relu=True, in_scale=0.02, algo="dot4", **kw)
    f1 = M.qconv2d_nhwc_i8_dequant(xd, wd_, bd, sd, relu=True, in_scale=0.02, algo="dot4", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
    np.testing.assert_array_equal(q0.cpu().numpy(), oracle.requant_i8(acc_want, bias, ws, 0.02, 1.0, False))
    np.testing.assert_array_equal(q1.cpu().numpy(), oracle.requant_i8(acc_want, None, ws, 0.02, 1.0, True))
    want_f = oracle.dequant_f32(acc_want, bias, ws, 0.02, 1.0, True)
    np.testing.assert_array_equal(f1.cpu().numpy().view(np.uint32), want_f.view(np.uint32))


def test_dot4_unaligned_output_and_input(device):
    """x one byte into its buffer (the byte gather) and y one byte into its own (scalar stores)."""
    n, h, wd, c, k = 1, 10, 12, 16, 16
    x = W.fill_i8_uniform(n * h * wd * c, 77, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * 9 * c, 78, -127, 127).reshape(k, 3, 3, c)
    ws = W.fill_f32_uniform(k, 79, 1e-3, 1e-2)
    xb = torch.zeros(x.size + 1, dtype=torch.int8, device=device)
    xb[1:] = torch.from_numpy(x.reshape(-1)).to(device)
    yb = torch.full((n * h * wd * k + 1,), 5, dtype=torch.int8, device=device)
    wd_, sd = torch.from_numpy(w).to(device), torch.from_numpy(ws).to(device)
    M.qconv2d_nhwc_i8(xb[1:].view(n, h, wd, c), wd_, None, sd, padding=1, in_scale=0.02, algo="dot4",
                      out=yb[1:].view(n, h, wd, k))
    torch.cuda.synchronize()
    want = oracle.requant_i8(oracle.conv_i8_acc(x, w, (1, 1, 1, 1, 1, 1, 1)), None, ws, 0.02, 1.0, False)
    np.testing.assert_array_equal(yb[1:].cpu().numpy().reshape(want.shape), want)
    assert int(yb[0]) == 5
