"""The virtual-pixel row-band kernel ("flat": stride 1, output pixels enumerated over rows
padded to the input halo's width, filter held in registers) against the CPU oracle.  The
shapes cover bands whose segment count leaves 0, 1, 2 or 3 tail segments (split by channel
block over the SIMDs, or rounded up to a junk main segment), bands too small for a main
segment, partly filled last bands, several chunk quads per pixel (two or three K-blocks per
tap), odd and even K-block counts (the two filter layouts in LDS), dilation, asymmetric
padding and padding wider than the filter reach, groups, several 64-channel tiles, narrow
and wide rows.  Integer outputs are bit-exact; the fp32 view is compared bit for bit
(tolerance 1 ulp, met with 0 ulp)."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W

pytestmark = pytest.mark.gpu

# (n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups))
SHAPES = [
    (2, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # the ResNet-50 3x3 layer's geometry, N=2
    (3, 11, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # Ho 11: a partly filled last band
    (2, 12, 12, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # narrow rows (L = 14)
    (1, 3, 3, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),       # one segment: tail chains only
    (1, 5, 7, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),       # a few segments
    (2, 9, 29, 64, 128, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # two channel tiles
    (1, 10, 100, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # wide rows (L = 102)
    (2, 13, 20, 128, 64, 1, 3, (0, 1, 1, 1, 1, 1, 1)),    # two quads per pixel, 1x3 taps (KB 6)
    (1, 14, 18, 64, 64, 3, 3, (2, 3, 1, 1, 2, 2, 1)),     # dilation 2, asymmetric padding
    (2, 6, 10, 64, 64, 3, 3, (4, 4, 1, 1, 1, 1, 1)),      # padding wider than the filter reach
    (1, 8, 8, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 2)),     # two groups of 64 channels
    (2, 9, 9, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),     # 1x1 (KB 2, fragment-order filter), 8 tiles
    (3, 7, 13, 64, 64, 1, 1, (0, 0, 1, 1, 1, 1, 1)),      # 1x1, KB 1
    (2, 17, 31, 192, 64, 1, 3, (0, 1, 1, 1, 1, 1, 1)),    # three quads per pixel (KB 9)
    (1, 9, 9, 64, 64, 1, 5, (0, 2, 1, 1, 1, 1, 1)),       # 1x5 taps (KB 5)
    (2, 15, 23, 64, 64, 2, 2, (0, 0, 1, 1, 1, 1, 1)),     # 2x2 taps (KB 4), no padding
    (4, 28, 28, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),   # the 1x1 expand layer's geometry, N=4
    # batches large enough for bands of several rows (several phases per wave):
    (16, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # 4-row bands: 3 tail segments -> a junk main one
    (6, 64, 64, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # 2-row bands: 2 main segments per SIMD + 1 tail
    (14, 41, 37, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # 3-row bands and a 2-row last band
    (9, 44, 60, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # 2-row bands, no tail
    (20, 25, 24, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # 3-row bands, a 1-row last band
    (16, 28, 28, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),  # 1x1 in multi-phase bands (two K-blocks per segment)
]


def _id(s):
    n, h, w, c, k, r, sz, conv = s
    return f"n{n}h{h}w{w}c{c}k{k}r{r}s{sz}p{conv[0]}{conv[1]}d{conv[4]}{conv[5]}g{conv[6]}"


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_flat_kernel_matches_oracle(device, shape):
    n, h, wd, c, k, r, s, conv = shape
    seed = 9100 + SHAPES.index(shape) * 16
    g = conv[6]
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * (c // g), seed + 1, -127, 127).reshape(k, r, s, c // g)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=g)
    assert M.plan(M.make_desc(x.shape, w.shape, algo="flat", **kw)) == "flat"
    assert M.plan(M.make_desc(x.shape, w.shape, **kw)) in ("band", "flat", "pointwise")  # auto
    acc_want = oracle.conv_i8_acc(x, w, conv)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    print(f"flat {_id(shape)}", flush=True)
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd_, algo="flat", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
    for relu in (False, True):
        q = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="flat", **kw)
        f = M.qconv2d_nhwc_i8_dequant(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="flat", **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, bias, ws, 0.02, 1.0, relu))
        want_f = oracle.dequant_f32(acc_want, bias, ws, 0.02, 1.0, relu)
        np.testing.assert_array_equal(f.cpu().numpy().view(np.uint32), want_f.view(np.uint32))
    q = M.qconv2d_nhwc_i8(xd, wd_, None, sd, in_scale=0.02, algo="flat", **kw)  # no bias: bias 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, None, ws, 0.02, 1.0, False))


def test_flat_rejects_what_it_cannot_run(device):
    x = torch.zeros((1, 8, 8, 64), dtype=torch.int8, device=device)
    for wshape, kw, msg in [((64, 3, 3, 64), dict(padding=1, stride=2), "stride 1"),
                            ((64, 3, 3, 32), dict(padding=1, groups=2), "% 64"),
                            ((48, 3, 3, 64), dict(padding=1), "% 64"),
                            ((64, 5, 5, 64), dict(padding=2), "registers")]:
        w = torch.zeros(wshape, dtype=torch.int8, device=device)
        with pytest.raises(M.MiqError, match=msg):
            M.qconv2d_nhwc_i8_acc32(x, w, algo="flat", **kw)
