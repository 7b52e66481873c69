"""The oracle's int32 batched matrix product (orc_bmm_i32, the semantics of the reference's
bmm_matmul_i32, /root/reference/bmm.cu:155-246 and :298-322), pinned without a GPU:

  - against numpy products in uint64 reduced modulo 2^32 (an independent evaluation: the
    two's-complement bit patterns multiply and add modulo 2^64, of which 2^32 is a divisor);
  - against brute-force Python integer loops on tiny inputs, all four transposes;
  - on known wrap-around answers (INT_MIN * -1, INT_MAX * INT_MAX, sums past 2^31);
  - at the reference's own call site (cuda_kernels.cu:1381: zero-point-corrected im2col
    columns times the packed filter with trans_b) against the reference's convolution
    accumulators held in the golden fixtures, which oracle/_ref's compiled cpu_ref.cpp wrote.

The reference has no test of its own for bmm_matmul_i32 (bmm_test.cu checks the fp32 bmm
only), so its call site in the quantized convolution is the anchor."""
import itertools

import numpy as np
import pytest

import oracle
from tests.golden import cases

INT_MIN, INT_MAX = -(2 ** 31), 2 ** 31 - 1


def numpy_bmm(a, b, ta, tb):
    a64 = (np.swapaxes(a, 1, 2) if ta else a).astype(np.int64).astype(np.uint64)
    b64 = (np.swapaxes(b, 1, 2) if tb else b).astype(np.int64).astype(np.uint64)
    return (a64 @ b64 & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.int32)


def operands(rng, batch, m, n, k, ta, tb, lo=INT_MIN, hi=INT_MAX):
    a = rng.integers(lo, hi, size=(batch, k, m) if ta else (batch, m, k), endpoint=True, dtype=np.int64)
    b = rng.integers(lo, hi, size=(batch, n, k) if tb else (batch, k, n), endpoint=True, dtype=np.int64)
    return a.astype(np.int32), b.astype(np.int32)


@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (3, 17, 9, 33), (2, 64, 128, 80), (1, 130, 70, 5), (4, 5, 6, 300)])
def test_bmm_matches_numpy_mod_2_32(shape, ta, tb):
    batch, m, n, k = shape
    rng = np.random.default_rng(hash((shape, ta, tb)) & 0xFFFF)
    a, b = operands(rng, batch, m, n, k, ta, tb)
    np.testing.assert_array_equal(oracle.bmm_i32(a, b, ta, tb), numpy_bmm(a, b, ta, tb))


@pytest.mark.parametrize("ta,tb", list(itertools.product([False, True], repeat=2)))
def test_bmm_brute_force_tiny(ta, tb):
    rng = np.random.default_rng(7 + 2 * ta + tb)
    batch, m, n, k = 2, 3, 4, 5
    a, b = operands(rng, batch, m, n, k, ta, tb)
    want = np.zeros((batch, m, n), np.int64)
    for bi in range(batch):
        for i in range(m):
            for j in range(n):
                s = 0
                for kk in range(k):
                    av = int(a[bi, kk, i] if ta else a[bi, i, kk])
                    bv = int(b[bi, j, kk] if tb else b[bi, kk, j])
                    s += av * bv
                s &= 0xFFFFFFFF
                want[bi, i, j] = s - (1 << 32) if s >= 1 << 31 else s
    np.testing.assert_array_equal(oracle.bmm_i32(a, b, ta, tb), want.astype(np.int32))


def test_bmm_wraparound_known_answers():
    a = np.array([[[INT_MIN], [INT_MAX], [INT_MAX], [-1]]], np.int32)       # 4 x 1
    b = np.array([[[-1, INT_MAX, INT_MIN, 1]]], np.int32)                    # 1 x 4
    c = oracle.bmm_i32(a, b)[0]
    assert c[0, 0] == INT_MIN           # INT_MIN * -1 wraps to INT_MIN
    assert c[1, 1] == 1                 # (2^31 - 1)^2 = 2^62 - 2^32 + 1 = 1 mod 2^32
    assert c[0, 2] == 0                 # 2^62 = 0 mod 2^32
    assert c[2, 2] == INT_MIN           # -(2^31 - 1) 2^31 = 2^31 mod 2^32
    assert c[3, 3] == -1
    k3 = oracle.bmm_i32(np.full((1, 1, 3), INT_MAX, np.int32), np.ones((1, 3, 1), np.int32))
    assert k3[0, 0, 0] == 2 ** 31 - 3   # 3 (2^31 - 1) = 2^32 + 2^31 - 3
    big = oracle.bmm_i32(np.full((1, 1, 200000), -128, np.int32), np.full((1, 200000, 1), -128, np.int32))
    assert big[0, 0, 0] == 200000 * 16384 - (1 << 32)   # 3276800000 is past 2^31


def test_bmm_empty_extents():
    assert oracle.bmm_i32(np.zeros((0, 3, 4), np.int32), np.zeros((0, 4, 5), np.int32)).shape == (0, 3, 5)
    assert oracle.bmm_i32(np.zeros((2, 0, 4), np.int32), np.zeros((2, 4, 5), np.int32)).shape == (2, 0, 5)
    c = oracle.bmm_i32(np.zeros((2, 3, 0), np.int32), np.zeros((2, 0, 5), np.int32))
    np.testing.assert_array_equal(c, np.zeros((2, 3, 5), np.int32))   # K == 0: zeros


def im2col_qi32(x, zp, r, s, conv, g, cg):
    """Zero-point-corrected columns of group g: rows (n, ho, wo), columns (r, s, c) - the
    matrix the reference's im2col kernel builds before its bmm call (cuda_kernels.cu:1365-1372)."""
    n, h, w, _ = x.shape
    ph, pw, sh, sw, dh, dw, _ = conv
    ho = (h + 2 * ph - dh * (r - 1) - 1) // sh + 1
    wo = (w + 2 * pw - dw * (s - 1) - 1) // sw + 1
    xi = x.astype(np.int32) - np.asarray(zp, np.int32).reshape(n, 1, 1, 1)
    col = np.zeros((n, ho, wo, r, s, cg), np.int32)
    for rr in range(r):
        for ss in range(s):
            for oh in range(ho):
                hi = oh * sh - ph + rr * dh
                if not 0 <= hi < h:
                    continue
                for ow in range(wo):
                    wi = ow * sw - pw + ss * dw
                    if 0 <= wi < w:
                        col[:, oh, ow, rr, ss, :] = xi[:, hi, wi, g * cg:(g + 1) * cg]
    return col.reshape(n * ho * wo, r * s * cg), (n, ho, wo)


def test_bmm_at_the_reference_call_site_reproduces_its_convolutions():
    ran = 0
    for name, c in cases.qi32_cases().items():
        if tuple(c["block"]) != (0, 0):
            continue
        x, w, conv = c["x"], c["w"], [int(v) for v in c["conv"]]
        k, r, s, cg = w.shape
        groups = conv[6]
        kg = k // groups
        y = np.zeros(c["y"].shape, np.int32)
        for g in range(groups):
            col, (n, ho, wo) = im2col_qi32(x, c["zp"], r, s, conv, g, cg)
            wg = (w[g * kg:(g + 1) * kg].astype(np.int32) - int(c["fzp"])).reshape(kg, r * s * cg)
            ym = oracle.bmm_i32(col[None], wg[None], trans_a=False, trans_b=True)[0]
            y[..., g * kg:(g + 1) * kg] = ym.reshape(n, ho, wo, kg)
        np.testing.assert_array_equal(y, c["y"], err_msg=name)
        ran += 1
    assert ran >= 4
