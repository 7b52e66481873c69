"""The oracle's blocked fp32 convolution (orc_block_conv_f32 / orc_block_bprop_f32 /
orc_block_grad_f32, the semantics of the reference's cpu_block_fprop_nhwc,
cpu_block_bprop_nhwc and cpu_block_grad_nhwc, /root/reference/src/cpu_ref.cpp:232-369),
pinned without a GPU:

  - bit for bit against the reference's own cpu_block_* compiled unmodified into
    oracle/_ref, over block grids, padding, stride, dilation, groups, both bias modes and
    dbias;
  - a 1 x 1 block grid against the dense oracle (the dense convolution is the special case);
  - against float64 torch autograd of the blocked operator written as a sum over blocks of
    a dense convolution masked to the block's output positions (a library routine), within
    fp32 rounding;
  - the shape rules: a block grid that does not divide Ho x Wo, or a zero grid, is rejected."""
import numpy as np
import pytest
import torch

import oracle

SHAPES = [  # n, h, w, c, k, r, s, conv7, by, bx
    (1, 8, 8, 8, 12, 3, 3, (1, 1, 1, 1, 1, 1, 1), 2, 2),
    (2, 12, 12, 16, 16, 3, 3, (1, 1, 1, 1, 1, 1, 1), 4, 4),
    (1, 14, 12, 8, 8, 3, 3, (1, 1, 2, 2, 1, 1, 1), 7, 2),        # stride 2, 7 x 6 output
    (2, 10, 10, 16, 16, 3, 3, (1, 1, 1, 1, 1, 1, 4), 2, 2),      # grouped
    (1, 8, 8, 8, 8, 3, 3, (1, 1, 1, 1, 1, 1, 8), 2, 4),          # depthwise
    (2, 8, 8, 24, 16, 1, 1, (0, 0, 1, 1, 1, 1, 1), 4, 4),        # pointwise
    (1, 12, 12, 8, 8, 3, 3, (2, 2, 1, 1, 2, 2, 1), 2, 2),        # dilated
    (1, 9, 9, 4, 6, 3, 3, (0, 0, 1, 1, 1, 1, 1), 7, 1),          # no padding, 7 x 7 output
    (1, 6, 10, 4, 4, 5, 3, (3, 2, 2, 3, 1, 1, 2), 2, 2),         # padding wider than the reach
]


def _data(shape, seed):
    n, h, w, c, k, r, s, conv, by, bx = shape
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, size=(n, h, w, c)).astype(np.float32)
    wt = rng.uniform(-1, 1, size=(k, by, bx, r, s, c // conv[6])).astype(np.float32)
    bias = rng.uniform(-1, 1, size=k * by * bx).astype(np.float32)
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    dy = rng.uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)
    return x, wt, bias, dy


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


needs_ref = pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref (the reference's cpu_ref.cpp) not built here")


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mode", [None, 0, 1])
def test_block_fprop_bit_exact_with_reference_cpu(shape, mode):
    x, wt, bias, _ = _data(shape, 11 + SHAPES.index(shape))
    b = None if mode is None else bias
    want, _, _ = oracle.ref_block_f32("fprop", x, wt, x.shape, wt.shape, shape[7], b, mode or 0)
    got = oracle.block_conv_f32(x, wt, shape[7], b, mode or 0)
    np.testing.assert_array_equal(_bits(got), _bits(want))


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
def test_block_bprop_bit_exact_with_reference_cpu(shape):
    x, wt, _, dy = _data(shape, 31 + SHAPES.index(shape))
    want, _, _ = oracle.ref_block_f32("bprop", dy, wt, x.shape, wt.shape, shape[7])
    np.testing.assert_array_equal(_bits(oracle.block_bprop_f32(dy, wt, x.shape, shape[7])), _bits(want))


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mode", [None, 0, 1])
def test_block_grad_bit_exact_with_reference_cpu(shape, mode):
    x, wt, _, dy = _data(shape, 51 + SHAPES.index(shape))
    k, by, bx = wt.shape[:3]
    # the reference accumulates into dbias after zeroing it: start from garbage to show the zeroing
    dbias_ref = None if mode is None else np.full(k * by * bx, 7.0, np.float32)
    want, _, dbias_ref = oracle.ref_block_f32("grad", x, dy, x.shape, wt.shape, shape[7], dbias_ref, mode or 0)
    if mode is None:
        got = oracle.block_grad_f32(x, dy, wt.shape, shape[7])
    else:
        got, dbias = oracle.block_grad_f32(x, dy, wt.shape, shape[7], with_dbias=True, bias_mode=mode)
        np.testing.assert_array_equal(_bits(dbias), _bits(dbias_ref))
    np.testing.assert_array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("shape", SHAPES)
def test_one_block_is_the_dense_convolution(shape):
    n, h, w, c, k, r, s, conv, _, _ = shape
    one = shape[:8] + (1, 1)
    x, wt, bias, dy = _data(one, 71 + SHAPES.index(shape))
    dense_w = wt[:, 0, 0]
    np.testing.assert_array_equal(_bits(oracle.block_conv_f32(x, wt, conv)), _bits(oracle.conv_f32(x, dense_w, conv)))
    np.testing.assert_array_equal(_bits(oracle.block_bprop_f32(dy, wt, x.shape, conv)),
                                  _bits(oracle.bprop_f32(dy, dense_w, x.shape, conv)))
    np.testing.assert_array_equal(_bits(oracle.block_grad_f32(x, dy, wt.shape, conv)[:, 0, 0]),
                                  _bits(oracle.grad_f32(x, dy, dense_w.shape, conv)))
    # bias is added once, after the tap sum: y + bias[k] rounded once
    with_bias = oracle.block_conv_f32(x, wt, conv, bias, 0)
    np.testing.assert_array_equal(_bits(with_bias), _bits(oracle.conv_f32(x, dense_w, conv) + bias[None, None, None, :]))


@pytest.mark.parametrize("shape", SHAPES)
def test_block_against_float64_autograd(shape):
    n, h, w, c, k, r, s, conv, by, bx = shape
    ph, pw, sh, sw, dh, dw, g = conv
    x, wt, bias, dy = _data(shape, 91 + SHAPES.index(shape))
    ho, wo = dy.shape[1:3]
    bho, bwo = ho // by, wo // bx
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 3, 1, 2).requires_grad_(True)
    wtt = torch.from_numpy(wt.astype(np.float64)).requires_grad_(True)
    xp = torch.nn.functional.pad(xt, (pw, pw, ph, ph))
    y = torch.zeros((n, k, ho, wo), dtype=torch.float64)
    for i in range(by):
        for j in range(bx):
            mask = torch.zeros((1, 1, ho, wo), dtype=torch.float64)
            mask[..., i * bho:(i + 1) * bho, j * bwo:(j + 1) * bwo] = 1
            yb = torch.nn.functional.conv2d(xp, wtt[:, i, j].permute(0, 3, 1, 2), stride=(sh, sw),
                                            dilation=(dh, dw), groups=g)
            y = y + mask * yb
    y.backward(torch.from_numpy(dy.astype(np.float64)).permute(0, 3, 1, 2))
    taps = r * s * (c // g)
    np.testing.assert_allclose(oracle.block_conv_f32(x, wt, conv), y.detach().permute(0, 2, 3, 1).numpy(), rtol=0,
                               atol=taps * taps * 2.0 ** -24 + 1e-6)
    terms_dx = r * s * (k // g)
    np.testing.assert_allclose(oracle.block_bprop_f32(dy, wt, x.shape, conv), xt.grad.permute(0, 2, 3, 1).numpy(),
                               rtol=0, atol=terms_dx * terms_dx * 2.0 ** -24 + 1e-6)
    terms_dw = n * bho * bwo
    np.testing.assert_allclose(oracle.block_grad_f32(x, dy, wt.shape, conv), wtt.grad.numpy(), rtol=0,
                               atol=terms_dw * terms_dw * 2.0 ** -24 + 1e-6)


@pytest.mark.parametrize("shape", SHAPES)
def test_dbias_counts_positions_with_the_first_tap_inside(shape):
    """dbias[k][by][bx] (PerBlock) sums dy over the block's output positions whose (r, s) =
    (0, 0) tap reads inside the image; Shared puts every block's sum into [k][0][0] and
    leaves the other slots zero."""
    n, h, w, c, k, r, s, conv, by, bx = shape
    ph, pw, sh, sw = conv[:4]
    x, wt, _, dy = _data(shape, 131 + SHAPES.index(shape))
    ho, wo = dy.shape[1:3]
    hi = np.arange(ho) * sh - ph
    wi = np.arange(wo) * sw - pw
    inside = ((hi >= 0) & (hi < h))[:, None] & ((wi >= 0) & (wi < w))[None, :]
    sums = (dy.astype(np.float64) * inside[None, :, :, None]).sum(axis=0)  # ho x wo x k
    per_block = sums.reshape(by, ho // by, bx, wo // bx, k).sum(axis=(1, 3)).transpose(2, 0, 1)  # k x by x bx
    _, db0 = oracle.block_grad_f32(x, dy, wt.shape, conv, with_dbias=True, bias_mode=0)
    np.testing.assert_allclose(db0.reshape(k, by, bx), per_block, rtol=0, atol=n * ho * wo * 2.0 ** -22)
    _, db1 = oracle.block_grad_f32(x, dy, wt.shape, conv, with_dbias=True, bias_mode=1)
    db1 = db1.reshape(k, by, bx)
    np.testing.assert_allclose(db1[:, 0, 0], per_block.sum(axis=(1, 2)), rtol=0, atol=n * ho * wo * 2.0 ** -22)
    db1[:, 0, 0] = 0
    assert not db1.any()


@pytest.mark.parametrize("by,bx", [(3, 2), (2, 3), (0, 2), (2, 0), (-1, 1)])
def test_block_grid_must_divide_output(by, bx):
    """8 x 8 output (3x3, pad 1): grids 3 x 2 and 2 x 3 do not divide it, zero or negative
    grids are rejected outright - by the oracle and by the reference alike."""
    import ctypes as C
    x = np.zeros((1, 8, 8, 4), np.float32)
    wt = np.zeros(4 * max(by, 1) * max(bx, 1) * 9 * 4, np.float32)
    y = np.zeros(1 * 8 * 8 * 4, np.float32)
    conv = oracle._conv7((1, 1, 1, 1, 1, 1, 1))
    p = oracle._p
    assert oracle.orc().orc_block_conv_f32(p(x), 1, 8, 8, 4, p(wt), 3, 3, 4, p(conv), by, bx, None, 0, p(y), 1) == -1
    assert oracle.orc().orc_block_bprop_f32(p(y), 1, 8, 8, 4, p(wt), 3, 3, 4, p(conv), by, bx, p(x), 1) == -1
    assert oracle.orc().orc_block_grad_f32(p(x), 1, 8, 8, 4, p(y), 3, 3, 4, p(conv), by, bx, p(wt), None, 0, 1) == -1
    with pytest.raises(ValueError):
        oracle._block_out_shape(1, 8, 8, 4, 3, 3, 4, conv, by, bx)
    h = oracle.ref()
    if h is not None:
        secs = C.c_double()
        for op in range(3):
            assert h.ref_block_f32(op, p(x), p(wt), 1, 8, 8, 4, 3, 3, 4, p(conv), by, bx, None, 0, p(y),
                                   C.byref(secs)) == -1


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mode", [0, 1])
def test_all_positions_dbias(shape, mode):
    """The library's bias gradient (every position of a block, as launch_block_grad_nhwc sums
    it) in its fixed run order: one run per block where every (0, 0) tap is inside (no padding)
    gives the reference CPU's dbias bit for bit in per-block mode; any run length stays within
    fp32 rounding of the float64 sum; with padding, it exceeds the CPU form by exactly the dy of
    the positions whose (0, 0) tap is in the padding."""
    n, h, w, c, k, r, s, conv, by, bx = shape
    x, wt, _, dy = _data(shape, 151 + SHAPES.index(shape))
    ho, wo = dy.shape[1:3]
    full = dy.astype(np.float64).reshape(n, by, ho // by, bx, wo // bx, k).sum(axis=(0, 2, 4)).transpose(2, 0, 1)
    if mode == 0:
        want = full
    else:
        want = np.zeros((k, by, bx))
        want[:, 0, 0] = full.sum(axis=(1, 2))
    for chunk in (0, 7, 256):
        got = oracle.block_dbias_f32(dy, by, bx, mode, chunk).reshape(k, by, bx)
        np.testing.assert_allclose(got, want, rtol=0, atol=n * ho * wo * 2.0 ** -22)
    if oracle.ref() is not None and mode == 0:
        noconv = (0, 0) + tuple(conv[2:])  # same geometry without padding
        ho0, wo0 = oracle.conv_output_shape(n, h, w, c, r, s, k, noconv)
        if ho0 % by == 0 and wo0 % bx == 0:
            dy0 = np.random.default_rng(7).uniform(-1, 1, size=(n, ho0, wo0, k)).astype(np.float32)
            _, _, cpu = oracle.ref_block_f32("grad", x, dy0, x.shape, wt.shape, noconv,
                                             np.zeros(k * by * bx, np.float32), 0)
            np.testing.assert_array_equal(_bits(oracle.block_dbias_f32(dy0, by, bx, 0, 0)), _bits(cpu))


def test_dbias_rules_differ_only_at_padded_first_taps():
    shape = SHAPES[0]  # 3x3, padding 1: output row 0 and column 0 read their (0, 0) tap in the padding
    n, h, w, c, k, r, s, conv, by, bx = shape
    x, wt, _, dy = _data(shape, 171)
    _, cpu = oracle.block_grad_f32(x, dy, wt.shape, conv, with_dbias=True, bias_mode=0)
    lib = oracle.block_dbias_f32(dy, by, bx, 0, 0)
    ho, wo = dy.shape[1:3]
    edge = np.zeros((ho, wo), bool)
    edge[0, :] = True
    edge[:, 0] = True
    skipped = (dy.astype(np.float64) * edge[None, :, :, None]).reshape(n, by, ho // by, bx, wo // bx, k)
    skipped = skipped.sum(axis=(0, 2, 4)).transpose(2, 0, 1).reshape(-1)
    np.testing.assert_allclose(lib.astype(np.float64) - cpu, skipped, rtol=0, atol=1e-5)
    assert np.abs(skipped).max() > 1e-3  # the rules really differ here
