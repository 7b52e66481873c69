"""The filter-streaming row-band kernel (input rows in LDS, the filter streamed through a
ring of K-block buffers) against the CPU oracle on the geometry classes it accepts:
stride 2 and 3 (column parity planes), stride 1 with filters too large for registers,
output widths above 64, rows whose packed 16-pixel segments wrap into the next row with
and without a bank-conflict-free row padding, 1x1 projections, dilation, groups, 5x5
taps, 128- and 256-channel workgroups, padding wider than the filter reach and a last
band that is only partly filled.  Integer outputs are bit-exact; the fp32 view is
compared bit for bit (tolerance 1 ulp, met with 0 ulp)."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W

pytestmark = pytest.mark.gpu

# (n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups))
SHAPES = [
    (2, 14, 14, 128, 256, 3, 3, (1, 1, 2, 2, 1, 1, 1)),   # the down_s2 layer shape, Wo 7
    (1, 20, 18, 64, 128, 3, 3, (1, 1, 2, 2, 1, 1, 1)),    # Wo 9 with stride 2: no conflict-free row padding
    (2, 9, 11, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # stride 1, 18 K-blocks (too many for registers)
    (1, 12, 70, 64, 128, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # Wo 70: five 16-column blocks per plane
    (2, 16, 16, 256, 256, 1, 1, (0, 0, 2, 2, 1, 1, 1)),   # 1x1 stride-2 projection
    (1, 13, 13, 64, 128, 3, 3, (2, 2, 1, 1, 2, 2, 1)),    # dilation 2
    (1, 11, 15, 128, 256, 3, 3, (1, 1, 2, 2, 1, 1, 2)),   # two groups of 64 -> 128 channels
    (3, 10, 10, 64, 128, 5, 5, (2, 2, 1, 1, 1, 1, 1)),    # 5x5 taps, 25 K-blocks
    (1, 15, 21, 64, 128, 3, 3, (3, 4, 3, 3, 1, 1, 1)),    # stride 3, padding wider than the filter reach
    (4, 8, 8, 64, 384, 3, 3, (1, 1, 1, 1, 1, 1, 1)),      # 384 channels: 128-channel workgroups
    (2, 30, 30, 128, 256, 3, 3, (1, 1, 2, 2, 1, 1, 1)),   # Ho 15: a partly filled last band
    (1, 7, 9, 192, 128, 1, 3, (0, 1, 1, 2, 1, 1, 1)),     # three chunk quads per tap, 1x3 taps, stride_w 2
]


def _id(s):
    n, h, w, c, k, r, sz, conv = s
    return f"n{n}h{h}w{w}c{c}k{k}r{r}s{sz}p{conv[0]}{conv[1]}s{conv[2]}{conv[3]}d{conv[4]}{conv[5]}g{conv[6]}"


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_stream_kernel_matches_oracle(device, shape):
    n, h, wd, c, k, r, s, conv = shape
    seed = 8100 + SHAPES.index(shape) * 16
    g = conv[6]
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * (c // g), seed + 1, -127, 127).reshape(k, r, s, c // g)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=g)
    assert M.plan(M.make_desc(x.shape, w.shape, algo="stream", **kw)) == "stream"
    acc_want = oracle.conv_i8_acc(x, w, conv)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd_, algo="stream", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
    for relu in (False, True):
        q = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="stream", **kw)
        f = M.qconv2d_nhwc_i8_dequant(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="stream", **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, bias, ws, 0.02, 1.0, relu))
        want_f = oracle.dequant_f32(acc_want, bias, ws, 0.02, 1.0, relu)
        np.testing.assert_array_equal(f.cpu().numpy().view(np.uint32), want_f.view(np.uint32))
    q = M.qconv2d_nhwc_i8(xd, wd_, None, sd, in_scale=0.02, algo="stream", **kw)  # no bias pointer: bias 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, None, ws, 0.02, 1.0, False))


def test_stream_rejects_what_it_cannot_run(device):
    x = torch.zeros((1, 8, 8, 64), dtype=torch.int8, device=device)
    for wshape, kw, msg in [((128, 3, 3, 32), dict(padding=1, groups=2), "% 64"),
                            ((64, 3, 3, 64), dict(padding=1), "% 128"),
                            ((128, 3, 3, 64), dict(padding=1, stride=(1, 5)), "stride_w")]:
        w = torch.zeros(wshape, dtype=torch.int8, device=device)
        with pytest.raises(M.MiqError, match=msg):
            M.qconv2d_nhwc_i8_acc32(x, w, algo="stream", **kw)
