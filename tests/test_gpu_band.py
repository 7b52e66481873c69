"""The row-band kernel (filter held in registers, input rows streamed into LDS) against the
CPU oracle on every geometry class it accepts: output widths that leave partial 16-pixel
segments (1 to 4 segment columns per row), 1, 2, 4 or 8 channel tiles per workgroup, a
last band of the image that is only partly filled, vertical stride and dilation, padding
wider than the filter reach, groups, several 64-channel tiles and a partial one, and
inputs whose rows need two 64-column loads.  Integer outputs are bit-exact; the fp32 view is compared
bit for bit (tolerance 1 ulp, met with 0 ulp)."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W

pytestmark = pytest.mark.gpu

# (n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups))
SHAPES = [
    (2, 12, 12, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # Wo 12: one segment column, 4 row phases
    (1, 9, 29, 64, 32, 3, 3, (1, 1, 1, 1, 1, 1, 1)),      # Wo 29: two columns, partial channel tile
    (2, 7, 40, 64, 48, 3, 3, (1, 1, 1, 1, 1, 1, 1)),      # Wo 40: three columns
    (3, 11, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # the r50 3x3 row shape, odd band split
    (1, 10, 64, 64, 80, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # Wo 64: rows of 66 columns, two loads each
    (2, 13, 20, 128, 64, 1, 3, (0, 1, 2, 1, 1, 1, 1)),    # stride_h 2, Cg16 = 8 (two K-blocks per tap)
    (1, 14, 18, 64, 64, 3, 3, (2, 3, 1, 1, 2, 2, 1)),     # dilation 2, asymmetric padding
    (2, 6, 10, 64, 64, 3, 3, (4, 4, 1, 1, 1, 1, 1)),      # padding wider than the filter reach
    (1, 8, 8, 128, 96, 3, 3, (1, 1, 1, 1, 1, 1, 2)),      # two groups of 64 channels
    (2, 5, 9, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),     # 1x1, eight channel tiles
    (1, 9, 9, 64, 16, 1, 5, (0, 2, 1, 1, 1, 1, 1)),       # 1x5 taps, 16 output channels
    (2, 17, 31, 192, 64, 1, 3, (0, 1, 1, 1, 1, 1, 1)),    # Cg16 = 12, 1x3 taps
]


# Larger problems, for which the planner puts 2, 4 or 8 64-channel tiles in a workgroup
# (fewer, fuller rounds) or bands of several rows whose last band is partly filled; the
# comment gives the plan (tiles per workgroup, segment columns, band rows / output rows).
SHAPES_TILES = [
    (4, 19, 12, 64, 256, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # 1 tile, 1 column, bands of 2 / 19 rows
    (4, 19, 40, 64, 256, 3, 3, (1, 1, 1, 1, 1, 1, 1)),    # 1 tile, 3 columns, 2 / 19
    (4, 13, 50, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),   # 1 tile, 4 columns, 2 / 13
    (8, 37, 12, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),   # 2 tiles, 1 column, 5 / 37
    (24, 19, 20, 64, 256, 3, 3, (1, 1, 1, 1, 1, 1, 1)),   # 2 tiles, 2 columns, 3x3, 4 / 19
    (8, 13, 40, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),   # 2 tiles, 3 columns, 2 / 13
    (24, 19, 12, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),  # 4 tiles, 1 column, 4 / 19
    (12, 28, 40, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),  # 4 tiles, 3 columns, 3 / 28
    (12, 28, 50, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),  # 4 tiles, 4 columns, 3 / 28
    (40, 30, 50, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1)),  # 8 tiles, 4 columns, 5 / 30
]


def _id(s):
    n, h, w, c, k, r, sz, conv = s
    return f"n{n}h{h}w{w}c{c}k{k}r{r}s{sz}p{conv[0]}{conv[1]}s{conv[2]}d{conv[4]}{conv[5]}g{conv[6]}"


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_band_kernel_matches_oracle(device, shape):
    check_band(device, shape, 7000 + SHAPES.index(shape) * 16)


@pytest.mark.parametrize("shape", SHAPES_TILES, ids=[_id(s) for s in SHAPES_TILES])
def test_band_kernel_tiles_per_workgroup(device, shape):
    check_band(device, shape, 7500 + SHAPES_TILES.index(shape) * 16)


def check_band(device, shape, seed):
    n, h, wd, c, k, r, s, conv = shape
    g = conv[6]
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * (c // g), seed + 1, -127, 127).reshape(k, r, s, c // g)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=g)
    d = M.make_desc(x.shape, w.shape, algo="band", **kw)
    assert M.plan(d) == "band"
    # what auto picks: the pointwise kernel for the 1x1 shapes it takes, else the band kernel
    pointwise = (r, s, g) == (1, 1, 1) and conv[:4] == (0, 0, 1, 1) and c in (64, 128) and k % 64 == 0
    assert M.plan(M.make_desc(x.shape, w.shape, **kw)) == ("pointwise" if pointwise else "band")
    acc_want = oracle.conv_i8_acc(x, w, conv)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd_, algo="band", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
    for relu in (False, True):
        q = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="band", **kw)
        f = M.qconv2d_nhwc_i8_dequant(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="band", **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, bias, ws, 0.02, 1.0, relu))
        want_f = oracle.dequant_f32(acc_want, bias, ws, 0.02, 1.0, relu)
        np.testing.assert_array_equal(f.cpu().numpy().view(np.uint32), want_f.view(np.uint32))
    # no bias pointer: bias 0
    q = M.qconv2d_nhwc_i8(xd, wd_, None, sd, in_scale=0.02, algo="band", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, None, ws, 0.02, 1.0, False))


def test_band_rejects_what_it_cannot_run(device):
    x = torch.zeros((1, 8, 8, 64), dtype=torch.int8, device=device)
    for wshape, kw, msg in [((64, 3, 3, 64), dict(padding=1, stride=2), "stride_w"),
                            ((64, 3, 3, 32), dict(padding=1, groups=2), "% 64"),
                            ((40, 3, 3, 64), dict(padding=1), "% 16"),
                            ((64, 5, 5, 64), dict(padding=2), "registers")]:
        w = torch.zeros(wshape, dtype=torch.int8, device=device)
        with pytest.raises(M.MiqError, match=msg):
            M.qconv2d_nhwc_i8_acc32(x, w, algo="band", **kw)
    wide = torch.zeros((1, 4, 80, 64), dtype=torch.int8, device=device)
    with pytest.raises(M.MiqError, match="width"):
        M.qconv2d_nhwc_i8_acc32(wide, torch.zeros((64, 3, 3, 64), dtype=torch.int8, device=device), padding=1,
                                algo="band")
