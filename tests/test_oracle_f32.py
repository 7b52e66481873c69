"""The oracle's fp32 convolution (orc_conv_f32, the semantics of the reference's
cpu_fprop_nhwc, /root/reference/src/cpu_ref.cpp:116-146) and its verify_tensors pass rule
(src/verify.cpp:7-36), pinned without a GPU:

  - bit for bit against the reference's own cpu_fprop_nhwc compiled unmodified into
    oracle/_ref (same loop order and fp32 operations), over padding, stride, dilation,
    groups, depthwise and 1x1 shapes;
  - against a float64 torch convolution (a library routine) within fp32 rounding;
  - the numpy restatement of verify_tensors against the reference's compiled one on
    vectors at and around both thresholds."""
import numpy as np
import pytest
import torch

import oracle

SHAPES = [  # n, h, w, c, k, r, s, conv7
    (1, 9, 11, 8, 12, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    (2, 12, 10, 16, 32, 3, 3, (1, 1, 2, 2, 1, 1, 1)),
    (1, 14, 14, 16, 16, 3, 3, (1, 1, 1, 1, 1, 1, 16)),    # depthwise
    (1, 13, 13, 32, 32, 3, 3, (1, 1, 1, 1, 1, 1, 4)),     # grouped
    (2, 8, 8, 24, 40, 1, 1, (0, 0, 1, 1, 1, 1, 1)),       # pointwise
    (1, 16, 16, 8, 8, 3, 3, (2, 2, 1, 1, 2, 2, 1)),       # dilated
    (1, 20, 17, 3, 8, 7, 7, (3, 3, 2, 2, 1, 1, 1)),       # stem-like
    (1, 5, 7, 4, 6, 5, 3, (4, 2, 3, 2, 1, 1, 2)),         # padding wider than the filter reach
]


def _data(shape, seed):
    n, h, w, c, k, r, s, conv = shape
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, size=(n, h, w, c)).astype(np.float32)
    wt = rng.uniform(-1, 1, size=(k, r, s, c // conv[6])).astype(np.float32)
    return x, wt


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref (the reference's cpu_ref.cpp) not built here")
@pytest.mark.parametrize("shape", SHAPES)
def test_conv_f32_bit_exact_with_reference_cpu(shape):
    x, wt = _data(shape, 11 + SHAPES.index(shape))
    want, _ = oracle.ref_conv_f32(x, wt, shape[7])
    got = oracle.conv_f32(x, wt, shape[7])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("shape", SHAPES)
def test_conv_f32_against_float64_torch(shape):
    x, wt = _data(shape, 31 + SHAPES.index(shape))
    ph, pw, sh, sw, dh, dw, g = shape[7]
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 3, 1, 2)
    wtt = torch.from_numpy(wt.astype(np.float64)).permute(0, 3, 1, 2)
    xt = torch.nn.functional.pad(xt, (pw, pw, ph, ph))
    ref = torch.nn.functional.conv2d(xt, wtt, stride=(sh, sw), dilation=(dh, dw), groups=g)
    ref = ref.permute(0, 2, 3, 1).numpy()
    got = oracle.conv_f32(x, wt, shape[7]).astype(np.float64)
    taps = shape[5] * shape[6] * (shape[3] // g)
    # sequential fp32 sum of `taps` products of magnitude <= 1: error <= taps^2 * 2^-24 loosely
    np.testing.assert_allclose(got, ref, rtol=0, atol=taps * taps * 2.0 ** -24 + 1e-6)


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref (the reference's cpu_ref.cpp) not built here")
def test_verify_rule_matches_reference():
    a = np.array([1.0, 1.0, 0.0, 0.0, 5e-7, 100.0, -2.0, 1e-3], np.float32)
    cases = [
        a,
        a + np.float32(9e-5),                                       # under abs_eps everywhere
        a + np.array([0, 2e-4, 0, 0, 0, 0, 0, 0], np.float32),      # abs > 1e-4 but rel 2e-4 < 1e-3
        a + np.array([0, 0, 2e-4, 0, 0, 0, 0, 0], np.float32),      # zero reference: abs alone decides
        a + np.array([0, 0, 0, 0, 0, 0.2, 0, 0], np.float32),       # rel 2e-3 on 100
        a + np.array([0, 0, 0, 0, 0, 0.05, 0, 0], np.float32),      # rel 5e-4 on 100
        a + np.array([0, 0, 0, 0, 2e-4, 0, 0, 0], np.float32),      # |a| <= 1e-6: fails on abs
        a + np.array([0, 0, 0, 0, 0, 0, -2.1e-3, 0], np.float32),   # rel just over 1e-3
    ]
    for got in cases:
        want = oracle.ref_verify_tensors(a, got, 1e-4, 1e-3)["passed"]
        assert oracle.verify_tensors(a, got) == want, got


def _dy(shape, seed):
    n, h, w, c, k, r, s, conv = shape
    ho_wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    return np.random.default_rng(seed).uniform(-1, 1, size=(n, ho_wo[0], ho_wo[1], k)).astype(np.float32)


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref (the reference's cpu_ref.cpp) not built here")
@pytest.mark.parametrize("shape", SHAPES)
def test_bprop_grad_f32_bit_exact_with_reference_cpu(shape):
    x, wt = _data(shape, 51 + SHAPES.index(shape))
    dy = _dy(shape, 71 + SHAPES.index(shape))
    conv = shape[7]
    want_dx, _ = oracle.ref_backward_f32("bprop", dy, wt, x.shape, wt.shape, conv)
    np.testing.assert_array_equal(oracle.bprop_f32(dy, wt, x.shape, conv).view(np.uint32), want_dx.view(np.uint32))
    want_dw, _ = oracle.ref_backward_f32("grad", x, dy, x.shape, wt.shape, conv)
    np.testing.assert_array_equal(oracle.grad_f32(x, dy, wt.shape, conv).view(np.uint32), want_dw.view(np.uint32))


@pytest.mark.parametrize("shape", SHAPES)
def test_bprop_grad_f32_against_float64_autograd(shape):
    x, wt = _data(shape, 91 + SHAPES.index(shape))
    dy = _dy(shape, 111 + SHAPES.index(shape))
    ph, pw, sh, sw, dh, dw, g = shape[7]
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 3, 1, 2).requires_grad_(True)
    wtt = torch.from_numpy(wt.astype(np.float64)).permute(0, 3, 1, 2).requires_grad_(True)
    y = torch.nn.functional.conv2d(torch.nn.functional.pad(xt, (pw, pw, ph, ph)), wtt, stride=(sh, sw),
                                   dilation=(dh, dw), groups=g)
    y.backward(torch.from_numpy(dy.astype(np.float64)).permute(0, 3, 1, 2))
    ref_dx = xt.grad.permute(0, 2, 3, 1).numpy()
    ref_dw = wtt.grad.permute(0, 2, 3, 1).numpy()
    terms_dx = shape[5] * shape[6] * (shape[4] // g)
    terms_dw = dy.shape[0] * dy.shape[1] * dy.shape[2]
    np.testing.assert_allclose(oracle.bprop_f32(dy, wt, x.shape, shape[7]), ref_dx, rtol=0,
                               atol=terms_dx * terms_dx * 2.0 ** -24 + 1e-6)
    np.testing.assert_allclose(oracle.grad_f32(x, dy, wt.shape, shape[7]), ref_dw, rtol=0,
                               atol=terms_dw * terms_dw * 2.0 ** -24 + 1e-6)
