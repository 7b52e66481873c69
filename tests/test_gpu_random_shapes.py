"""A seeded sweep of random convolution shapes: for each, the AUTO choice and every kernel
family that accepts the shape (row band, virtual-pixel band, filter stream, implicit GEMM, stem, direct) against
the CPU oracle (the vector-ALU dot4 kernel included).  The shapes draw channel counts, filter sizes, strides, padding, dilation and
groups at random within small sizes, so the planners' choices (tiles per workgroup, ring
depths, odd and even K-block counts, band heights, partly filled bands and segments) vary
from shape to shape.  Integer outputs bit-exact; the fp32 view bit for bit."""
import random

import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from my_own_cnn_amd import workloads as W

pytestmark = pytest.mark.gpu

ALGOS = ["band", "flat", "stream", "igemm", "stem", "dot4", "direct"]


def _shapes(count, seed):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        g = rng.choice([1, 1, 1, 2])
        cg = rng.choice([3, 16, 32, 64, 64, 128, 192]) if g == 1 else rng.choice([16, 64, 128])
        kg = rng.choice([16, 32, 64, 128, 128, 256, 384])
        r, s = rng.choice([(1, 1), (3, 3), (3, 3), (1, 3), (5, 5), (7, 7)])
        sh, sw = rng.choice([(1, 1), (1, 1), (2, 2), (1, 2), (2, 1), (3, 3)])
        dh, dw = rng.choice([(1, 1), (1, 1), (1, 1), (2, 2)])
        ph, pw = rng.randint(0, r), rng.randint(0, s)
        n = rng.randint(1, 3)
        h, w = rng.randint(max(1, (r - 1) * dh + 1 - 2 * ph), 24), rng.randint(max(1, (s - 1) * dw + 1 - 2 * pw), 40)
        ho = (h + 2 * ph - (r - 1) * dh - 1) // sh + 1
        wo = (w + 2 * pw - (s - 1) * dw - 1) // sw + 1
        if ho < 1 or wo < 1 or cg == 3 and g != 1:
            continue
        out.append((n, h, w, cg * g, kg * g, r, s, (ph, pw, sh, sw, dh, dw, g)))
    return out


SHAPES = _shapes(40, 20261202)


def _id(s):
    n, h, w, c, k, r, sz, conv = s
    return f"n{n}h{h}w{w}c{c}k{k}r{r}s{sz}p{conv[0]}{conv[1]}s{conv[2]}{conv[3]}d{conv[4]}{conv[5]}g{conv[6]}"


@pytest.mark.parametrize("shape", SHAPES, ids=[_id(s) for s in SHAPES])
def test_random_shape_every_accepting_kernel(device, shape):
    n, h, wd, c, k, r, s, conv = shape
    seed = 9000 + SHAPES.index(shape) * 16
    g = conv[6]
    x = W.fill_i8_uniform(n * h * wd * c, seed, -128, 127).reshape(n, h, wd, c)
    w = W.fill_i8_uniform(k * r * s * (c // g), seed + 1, -127, 127).reshape(k, r, s, c // g)
    bias = W.fill_i32_uniform(k, seed + 2, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 3, 1e-3, 1e-2)
    kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=g)
    acc_want = oracle.conv_i8_acc(x, w, conv)
    q_want = {relu: oracle.requant_i8(acc_want, bias, ws, 0.02, 1.0, relu) for relu in (False, True)}
    f_want = oracle.dequant_f32(acc_want, bias, ws, 0.02, 1.0, True)
    xd, wd_, bd, sd = (torch.from_numpy(a).to(device) for a in (x, w, bias, ws))
    ran = []
    for algo in ["auto"] + ALGOS:
        try:
            M.plan(M.make_desc(x.shape, w.shape, algo=algo, **kw))
        except M.MiqError:
            continue  # this family does not take the shape
        acc = M.qconv2d_nhwc_i8_acc32(xd, wd_, algo=algo, **kw)
        q0 = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=False, in_scale=0.02, algo=algo, **kw)
        q1 = M.qconv2d_nhwc_i8(xd, wd_, bd, sd, relu=True, in_scale=0.02, algo=algo, **kw)
        f1 = M.qconv2d_nhwc_i8_dequant(xd, wd_, bd, sd, relu=True, in_scale=0.02, algo=algo, **kw)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(acc.cpu().numpy(), acc_want, err_msg=algo)
        np.testing.assert_array_equal(q0.cpu().numpy(), q_want[False], err_msg=algo)
        np.testing.assert_array_equal(q1.cpu().numpy(), q_want[True], err_msg=algo)
        np.testing.assert_array_equal(f1.cpu().numpy().view(np.uint32), f_want.view(np.uint32), err_msg=algo)
        ran.append(algo)
    assert "auto" in ran and "direct" in ran, ran

