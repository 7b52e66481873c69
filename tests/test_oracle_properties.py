"""The oracle against what the mathematics fixes: float64 convolution (exact for these
integer magnitudes), brute force on tiny inputs, and convolution identities chosen so
that a dropped term, a wrong sign or index, or a transposed operand fails one of them."""
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def torch_conv_f64(x_nhwc, w_krsc, conv):
    """Cross-correlation in float64 via torch (NCHW / KCRS)."""
    ph, pw, sh, sw, dh, dw, g = conv
    x = torch.from_numpy(np.asarray(x_nhwc, np.float64)).permute(0, 3, 1, 2)
    w = torch.from_numpy(np.asarray(w_krsc, np.float64)).permute(0, 3, 1, 2)
    y = F.conv2d(x, w, stride=(sh, sw), padding=(ph, pw), dilation=(dh, dw), groups=g)
    return y.permute(0, 2, 3, 1).numpy()


def rand_case(rng, groups=None):
    g = groups or int(rng.choice([1, 2, 4]))
    cg, kg = int(rng.integers(1, 9)), int(rng.integers(1, 6))
    n, h, w = int(rng.integers(1, 4)), int(rng.integers(3, 12)), int(rng.integers(3, 12))
    r, s = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    conv = (int(rng.integers(0, 3)), int(rng.integers(0, 3)), int(rng.integers(1, 3)), int(rng.integers(1, 3)),
            int(rng.integers(1, 3)), int(rng.integers(1, 3)), g)
    x = rng.integers(-128, 128, size=(n, h, w, cg * g)).astype(np.int8)
    wt = rng.integers(-128, 128, size=(kg * g, r, s, cg)).astype(np.int8)
    return x, wt, conv


def test_int8_against_float64_conv():
    rng = np.random.default_rng(1)
    done = 0
    while done < 40:
        x, wt, conv = rand_case(rng)
        n, h, w, c = x.shape
        k, r, s, _ = wt.shape
        if oracle.conv_output_shape(n, h, w, c, r, s, k, conv) is None:
            continue
        got = oracle.conv_i8_acc(x, wt, conv)
        want = torch_conv_f64(x, wt, conv)
        np.testing.assert_array_equal(got, want.astype(np.int64))
        done += 1


def test_zero_points_against_float64_conv():
    # centring then zero padding == skipping padded taps with centred values
    rng = np.random.default_rng(2)
    for _ in range(20):
        x8, wt8, conv = rand_case(rng)
        x = (x8.astype(np.int32) + 128).astype(np.float32)  # uint8 codes
        wt = (wt8.astype(np.int32) + 128).astype(np.float32)
        zp = rng.integers(0, 256, size=x.shape[0]).astype(np.int32)
        fzp = int(rng.integers(0, 256))
        if oracle.conv_output_shape(*x.shape, *wt.shape[:3], conv) is None:
            continue
        got = oracle.conv_qi32(x, wt, conv, zp, fzp)
        want = torch_conv_f64(x - zp[:, None, None, None], wt - fzp, conv)
        np.testing.assert_array_equal(got, want.astype(np.int64))


def brute(x, wt, conv, zp, fzp):
    ph, pw, sh, sw, dh, dw, g = conv
    n, h, w, c = x.shape
    k, r, s, cg = wt.shape
    ho, wo = (h + 2 * ph - dh * (r - 1) - 1) // sh + 1, (w + 2 * pw - dw * (s - 1) - 1) // sw + 1
    kg = k // g
    y = np.zeros((n, ho, wo, k), np.int64)
    for ni, i, j, kk in itertools.product(range(n), range(ho), range(wo), range(k)):
        gi = kk // kg
        t = 0
        for a, b, ci in itertools.product(range(r), range(s), range(cg)):
            hi, wi = i * sh - ph + a * dh, j * sw - pw + b * dw
            if 0 <= hi < h and 0 <= wi < w:
                t += (int(x[ni, hi, wi, gi * cg + ci]) - zp[ni]) * (int(wt[kk, a, b, ci]) - fzp)
        y[ni, i, j, kk] = t
    return y


@pytest.mark.parametrize("conv", [(1, 0, 1, 1, 1, 1, 2), (0, 2, 2, 1, 1, 2, 1), (2, 1, 1, 2, 2, 1, 1)])
def test_brute_force_tiny(conv):
    rng = np.random.default_rng(3)
    g = conv[6]
    x = rng.integers(0, 20, size=(2, 5, 6, 2 * g)).astype(np.float32)
    wt = rng.integers(0, 20, size=(2 * g, 2, 3, 2)).astype(np.float32)
    zp, fzp = np.array([3, 11], np.int32), 7
    np.testing.assert_array_equal(oracle.conv_qi32(x, wt, conv, zp, fzp), brute(x, wt, conv, zp, fzp))


def test_truncation_toward_zero():
    # a single tap: y = trunc(x) * trunc(w) for codes of both signs
    x = np.array([2.9, -2.9, 0.5, -0.5], np.float32).reshape(4, 1, 1, 1)
    wt = np.array([-3.7], np.float32).reshape(1, 1, 1, 1)
    y = oracle.conv_qi32(x, wt, (0, 0, 1, 1, 1, 1, 1), np.zeros(4, np.int32), 0)
    np.testing.assert_array_equal(y.reshape(-1), [2 * -3, -2 * -3, 0, 0])


def test_stride_is_subsampled_stride_one():
    rng = np.random.default_rng(4)
    x = rng.integers(-128, 128, size=(2, 13, 11, 16)).astype(np.int8)
    wt = rng.integers(-128, 128, size=(8, 3, 3, 16)).astype(np.int8)
    full = oracle.conv_i8_acc(x, wt, (1, 1, 1, 1, 1, 1, 1))
    s2 = oracle.conv_i8_acc(x, wt, (1, 1, 2, 2, 1, 1, 1))
    np.testing.assert_array_equal(s2, full[:, ::2, ::2, :])


@pytest.mark.parametrize("dil", [(-1, -1), (1, -1), (-1, 1), (-2, 1)])
def test_negative_dilation_is_flipped_filter(dil):
    """dilation -d on an axis walks the taps backwards: hi = ho*sh - ph - d*r.  Flipping the
    filter along that axis and padding by ph + d*(R-1) gives the same taps with dilation +d
    (and the same output extent), which the float64 convolution pins."""
    rng = np.random.default_rng(12)
    x = rng.integers(-128, 128, size=(2, 7, 9, 6)).astype(np.int8)
    wt = rng.integers(-128, 128, size=(5, 3, 2, 6)).astype(np.int8)
    dh, dw = dil
    ph, pw = 1, 1
    got = oracle.conv_i8_acc(x, wt, (ph, pw, 1, 1, dh, dw, 1))
    wf = wt[:, ::-1] if dh < 0 else wt
    wf = wf[:, :, ::-1] if dw < 0 else wf
    ph2 = ph + (-dh) * (wt.shape[1] - 1) if dh < 0 else ph
    pw2 = pw + (-dw) * (wt.shape[2] - 1) if dw < 0 else pw
    want = torch_conv_f64(x, np.ascontiguousarray(wf), (ph2, pw2, 1, 1, abs(dh), abs(dw), 1))
    # torch pads symmetrically: keep the first Ho x Wo outputs (those hi = ho - ph2 + ...)
    np.testing.assert_array_equal(got, want[:, :got.shape[1], :got.shape[2]].astype(np.int64))
    if oracle.ref() is not None:
        xf, wff = x.astype(np.float32), wt.astype(np.float32)
        ref, _ = oracle.ref_conv_qi32("s5", xf, wff, (ph, pw, 1, 1, dh, dw, 1), np.zeros(2, np.int32), 0)
        np.testing.assert_array_equal(got, ref)


def test_padding_equals_explicit_zero_border():
    rng = np.random.default_rng(5)
    x = rng.integers(-128, 128, size=(1, 7, 9, 4)).astype(np.int8)
    wt = rng.integers(-128, 128, size=(5, 3, 2, 4)).astype(np.int8)
    xp = np.zeros((1, 7 + 4, 9 + 2, 4), np.int8)
    xp[:, 2:9, 1:10, :] = x
    np.testing.assert_array_equal(oracle.conv_i8_acc(x, wt, (2, 1, 1, 1, 1, 1, 1)),
                                  oracle.conv_i8_acc(xp, wt, (0, 0, 1, 1, 1, 1, 1)))


def test_groups_are_block_diagonal():
    rng = np.random.default_rng(6)
    g, cg, kg = 3, 4, 2
    x = rng.integers(-128, 128, size=(2, 6, 6, g * cg)).astype(np.int8)
    wt = rng.integers(-128, 128, size=(g * kg, 3, 3, cg)).astype(np.int8)
    y = oracle.conv_i8_acc(x, wt, (1, 1, 1, 1, 1, 1, g))
    for gi in range(g):
        part = oracle.conv_i8_acc(np.ascontiguousarray(x[..., gi * cg:(gi + 1) * cg]),
                                  np.ascontiguousarray(wt[gi * kg:(gi + 1) * kg]), (1, 1, 1, 1, 1, 1, 1))
        np.testing.assert_array_equal(y[..., gi * kg:(gi + 1) * kg], part)


def test_linearity_in_input():
    rng = np.random.default_rng(7)
    a = rng.integers(-64, 64, size=(1, 8, 8, 16)).astype(np.int8)
    b = rng.integers(-64, 64, size=(1, 8, 8, 16)).astype(np.int8)
    wt = rng.integers(-128, 128, size=(4, 3, 3, 16)).astype(np.int8)
    conv = (1, 1, 1, 1, 1, 1, 1)
    np.testing.assert_array_equal(oracle.conv_i8_acc((a + b).astype(np.int8), wt, conv),
                                  oracle.conv_i8_acc(a, wt, conv) + oracle.conv_i8_acc(b, wt, conv))


def test_zero_point_expansion_identity():
    # sum (x-zx)(w-zw) = sum xw - zw sum x - zx sum w + zx zw |taps|, over in-bounds taps
    rng = np.random.default_rng(8)
    x = rng.integers(0, 256, size=(2, 6, 7, 3)).astype(np.float32)
    wt = rng.integers(0, 256, size=(4, 3, 3, 3)).astype(np.float32)
    conv = (1, 1, 1, 1, 1, 1, 1)
    zp, fzp = np.array([17, 200], np.int32), 91
    lhs = oracle.conv_qi32(x, wt, conv, zp, fzp).astype(np.int64)
    z2 = np.zeros(2, np.int32)
    xw = oracle.conv_qi32(x, wt, conv, z2, 0).astype(np.int64)
    x1 = oracle.conv_qi32(x, np.ones_like(wt), conv, z2, 0).astype(np.int64)       # sum x over taps
    w1 = oracle.conv_qi32(np.ones_like(x), wt, conv, z2, 0).astype(np.int64)       # sum w over in-bounds taps
    cnt = oracle.conv_qi32(np.ones_like(x), np.ones_like(wt), conv, z2, 0).astype(np.int64)
    zx = zp[:, None, None, None].astype(np.int64)
    np.testing.assert_array_equal(lhs, xw - fzp * x1 - zx * w1 + zx * fzp * cnt)


def test_blocked_with_identical_blocks_is_regular():
    rng = np.random.default_rng(9)
    x = rng.integers(0, 256, size=(1, 6, 6, 4)).astype(np.float32)
    w1 = rng.integers(0, 256, size=(5, 3, 3, 4)).astype(np.float32)
    wb = np.broadcast_to(w1[:, None, None], (5, 2, 3, 3, 3, 4)).copy()
    zp = np.array([37], np.int32)
    conv = (1, 1, 1, 1, 1, 1, 1)
    np.testing.assert_array_equal(oracle.conv_qi32(x, wb, conv, zp, 91, (2, 3)), oracle.conv_qi32(x, w1, conv, zp, 91))


def test_blocked_selects_filter_by_output_block():
    rng = np.random.default_rng(10)
    x = rng.integers(-15, 16, size=(2, 6, 6, 4)).astype(np.float32)
    wb = rng.integers(-15, 16, size=(5, 2, 3, 3, 3, 4)).astype(np.float32)
    zp = np.array([-5, 2], np.int32)
    conv = (1, 1, 1, 1, 1, 1, 1)
    y = oracle.conv_qi32(x, wb, conv, zp, 3, (2, 3))
    for by in range(2):
        for bx in range(3):
            full = oracle.conv_qi32(x, np.ascontiguousarray(wb[:, by, bx]), conv, zp, 3)
            np.testing.assert_array_equal(y[:, by * 3:(by + 1) * 3, bx * 2:(bx + 1) * 2],
                                          full[:, by * 3:(by + 1) * 3, bx * 2:(bx + 1) * 2])


def test_output_channel_order_and_filter_layout():
    # one-hot filters pick single input taps: pins KRSC indexing and the g*Kg+ko order
    x = np.arange(1 * 4 * 4 * 4, dtype=np.float32).reshape(1, 4, 4, 4)
    wt = np.zeros((4, 3, 3, 2), np.float32)
    wt[0, 0, 0, 0] = 1   # group 0, tap (0,0), channel 0
    wt[1, 2, 1, 1] = 1   # group 0, tap (2,1), channel 1
    wt[2, 1, 2, 0] = 1   # group 1, tap (1,2), channel 2
    wt[3, 1, 1, 1] = 1   # group 1, centre tap, channel 3
    y = oracle.conv_qi32(x, wt, (1, 1, 1, 1, 1, 1, 2), np.zeros(1, np.int32), 0)
    xp = np.pad(x, ((0, 0), (1, 1), (1, 1), (0, 0)))
    np.testing.assert_array_equal(y[0, :, :, 0], xp[0, 0:4, 0:4, 0])
    np.testing.assert_array_equal(y[0, :, :, 1], xp[0, 2:6, 1:5, 1])
    np.testing.assert_array_equal(y[0, :, :, 2], xp[0, 1:5, 2:6, 2])
    np.testing.assert_array_equal(y[0, :, :, 3], x[0, :, :, 3])
