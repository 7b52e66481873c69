"""The row-band variant of the thin-channel kernel (bands of output rows, input rows and
the filter slice loaded straight into LDS, the filter held in registers) against the CPU
oracle.  It runs for every thin-channel shape whose input rows are whole 16-byte chunks
(W*C % 16 == 0) and whose channel count is whole 64-channel tiles; the shapes cover one and
two 16-byte slots per filter row (S*C <= 16 and <= 32), one to four K-blocks, bands of more
than one output row with a partly filled last band, partial 16-pixel segments, vertical
stride and dilation, asymmetric padding, horizontal stride 3 and several channel tiles.
Integer outputs are bit-exact; the fp32 view is compared bit for bit (tolerance 1 ulp, met
with 0 ulp)."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W

pytestmark = pytest.mark.gpu

# (n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups))
SHAPES = [
    (8, 110, 112, 3, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1)),   # the stem's rows; bands of 2 rows, last one partial
    (6, 100, 80, 3, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1)),    # Wo 40: a partial segment per row; 2-row bands
    (2, 48, 32, 3, 128, 7, 7, (3, 3, 2, 2, 1, 1, 1)),    # two channel tiles
    (2, 32, 32, 4, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),     # S*C = 12: one slot per row, one K-block
    (1, 20, 16, 1, 64, 5, 5, (2, 2, 1, 1, 1, 1, 1)),     # one channel
    (2, 19, 16, 8, 64, 3, 4, (0, 2, 2, 1, 2, 1, 1)),     # S*C = 32, stride_h 2, dilation_h 2
    (1, 9, 64, 2, 192, 1, 1, (0, 0, 1, 1, 1, 1, 1)),     # 1x1, three channel tiles, Wo 64
    (3, 40, 16, 15, 64, 2, 2, (1, 0, 1, 1, 1, 1, 1)),    # fifteen channels, S*C = 30
    (1, 7, 80, 5, 64, 3, 6, (1, 3, 1, 3, 1, 1, 1)),      # stride_w 3
]


def _id(s):
    n, h, w, c, k, r, sz, conv = s
    return f"n{n}h{h}w{w}c{c}k{k}r{r}s{sz}p{conv[0]}{conv[1]}s{conv[2]}{conv[3]}d{conv[4]}"


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_stem_band_matches_oracle(device, shape):
    n, h, wd, c, k, r, s, conv = shape
    assert (wd * c) % 16 == 0 and k % 64 == 0 and s * c <= 32  # the band variant's conditions
    seed = 9100 + SHAPES.index(shape) * 16
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * c, seed + 1, -127, 127).reshape(k, r, s, c)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]))
    # what auto picks: the space-to-depth kernel for stride-2 shapes with c <= 4, else this one
    s2d = conv[2:4] == (2, 2) and conv[4:6] == (1, 1) and c <= 4 and ((r + 1) // 2) * ((s + 1) // 2) <= 16
    assert M.plan(M.make_desc(x.shape, w.shape, **kw)) == ("stem_s2d" if s2d else "stem")
    acc_want = oracle.conv_i8_acc(x, w, conv)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd_, algo="stem", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
    for relu in (False, True):
        q = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="stem", **kw)
        f = M.qconv2d_nhwc_i8_dequant(xd, wd_, bd, sd, relu=relu, in_scale=0.02, algo="stem", **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, bias, ws, 0.02, 1.0, relu))
        want_f = oracle.dequant_f32(acc_want, bias, ws, 0.02, 1.0, relu)
        np.testing.assert_array_equal(f.cpu().numpy().view(np.uint32), want_f.view(np.uint32))
    q = M.qconv2d_nhwc_i8(xd, wd_, None, sd, in_scale=0.02, algo="stem", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(acc_want, None, ws, 0.02, 1.0, False))
