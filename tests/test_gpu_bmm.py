"""The int32 batched matrix product on the GPU (miq_bmm_i32 / bmm_matmul_i32, the MFMA
digit-product kernel) against the oracle's orc_bmm_i32, bit-exact: all four transposes,
extents that are not multiples of the 128 x 64 output tile or of the 16-value K chunk,
full-range int32 inputs, digit extremes (every base-256 digit -128 or 127), sums that wrap
past 2^31 in every shift group, K == 0, batches split over several launches, misaligned
output rows and the reference's own call site (im2col columns x packed filter, trans_b)."""
import itertools

import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle

pytestmark = pytest.mark.gpu

INT_MIN, INT_MAX = -(2 ** 31), 2 ** 31 - 1


def _operands(seed, batch, m, n, k, ta, tb, lo=INT_MIN, hi=INT_MAX):
    rng = np.random.default_rng(seed)
    a = rng.integers(lo, hi, size=(batch, k, m) if ta else (batch, m, k), endpoint=True, dtype=np.int64)
    b = rng.integers(lo, hi, size=(batch, n, k) if tb else (batch, k, n), endpoint=True, dtype=np.int64)
    return a.astype(np.int32), b.astype(np.int32)


def _run(device, a, b, ta, tb):
    ad, bd = torch.from_numpy(a).to(device), torch.from_numpy(b).to(device)
    c = M.bmm_i32(ad, bd, trans_a=ta, trans_b=tb)
    torch.cuda.synchronize()
    return c.cpu().numpy()


SHAPES = [  # batch, M, N, K
    (1, 1, 1, 1),
    (3, 17, 9, 33),
    (1, 128, 64, 16),      # exactly one tile and one chunk
    (2, 129, 65, 17),      # one past the tile and the chunk in every extent
    (2, 130, 70, 5),
    (1, 300, 200, 1000),
    (5, 7, 300, 64),
    (1, 256, 512, 640),
]
TRANS = list(itertools.product([False, True], repeat=2))


@pytest.mark.parametrize("ta,tb", TRANS)
@pytest.mark.parametrize("shape", SHAPES, ids=["b{}m{}n{}k{}".format(*s) for s in SHAPES])
def test_bmm_full_range_matches_oracle(device, shape, ta, tb):
    batch, m, n, k = shape
    a, b = _operands(1000 + SHAPES.index(shape) * 4 + 2 * ta + tb, batch, m, n, k, ta, tb)
    np.testing.assert_array_equal(_run(device, a, b, ta, tb), oracle.bmm_i32(a, b, ta, tb))


@pytest.mark.parametrize("ta,tb", TRANS)
def test_bmm_digit_extremes_and_int_limits(device, ta, tb):
    # 0x7F7F7F80 has every balanced digit -128, 0x7F7F7F7F every digit 127 with carries
    special = np.array([INT_MIN, INT_MAX, -1, 0, 1, 0x7F7F7F80, 0x7F7F7F7F, -0x7F7F7F80, 0x00808080, -0x00808080,
                        0x80, -0x80, 0x7F, 0x8080, 0x808080], np.int64).astype(np.int32)
    rng = np.random.default_rng(77 + 2 * ta + tb)
    batch, m, n, k = 2, 70, 90, 45
    a = special[rng.integers(0, special.size, size=(batch, k, m) if ta else (batch, m, k))]
    b = special[rng.integers(0, special.size, size=(batch, n, k) if tb else (batch, k, n))]
    np.testing.assert_array_equal(_run(device, a, b, ta, tb), oracle.bmm_i32(a, b, ta, tb))


def test_bmm_wraps_in_every_shift_group(device):
    # every digit -128: each of the four digit-product sums exceeds 2^31 in magnitude
    k = 200000
    a = np.full((1, 16, k), 0x7F7F7F80, np.int32)
    b = np.full((1, k, 20), 0x7F7F7F80, np.int32)
    b[0, ::3, 5] = INT_MIN
    got = _run(device, a, b, False, False)
    want = oracle.bmm_i32(a, b)
    np.testing.assert_array_equal(got, want)
    assert len(np.unique(want)) == 2


def test_bmm_k_zero_writes_zeros(device):
    c = torch.full((3, 40, 70), 12345, dtype=torch.int32, device=device)
    a = torch.empty((3, 40, 0), dtype=torch.int32, device=device)
    b = torch.empty((3, 0, 70), dtype=torch.int32, device=device)
    M.bmm_i32(a, b, out=c)
    torch.cuda.synchronize()
    assert int(c.abs().max()) == 0


def test_bmm_empty_extents_are_no_ops(device):
    for shape_a, shape_b in [((0, 5, 6), (0, 6, 7)), ((2, 0, 6), (2, 6, 7)), ((2, 5, 6), (2, 6, 0))]:
        a = torch.ones(shape_a, dtype=torch.int32, device=device)
        b = torch.ones(shape_b, dtype=torch.int32, device=device)
        assert M.bmm_i32(a, b).numel() == 0
    torch.cuda.synchronize()


def test_bmm_batch_split_over_launches(device):
    # 5,000,000 1x1 products: more workgroups than one launch takes (2^22)
    batch = 5_000_000
    a, b = _operands(4242, batch, 1, 1, 3, False, False)
    np.testing.assert_array_equal(_run(device, a, b, False, False), oracle.bmm_i32(a, b))


def test_bmm_misaligned_output_and_inputs(device):
    a, b = _operands(99, 2, 33, 36, 50, False, True)
    buf = torch.zeros(2 * 33 * 36 + 3, dtype=torch.int32, device=device)
    abuf = torch.zeros(a.size + 1, dtype=torch.int32, device=device)
    bbuf = torch.zeros(b.size + 1, dtype=torch.int32, device=device)
    abuf[1:] = torch.from_numpy(a.ravel()).to(device)
    bbuf[1:] = torch.from_numpy(b.ravel()).to(device)
    out = buf[1:1 + 2 * 33 * 36]  # 4-byte aligned only: the 16-byte store path is off
    M.bmm_matmul_i32(abuf[1:], bbuf[1:], out, 2, 33, 36, 50, 0, 1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().reshape(2, 33, 36), oracle.bmm_i32(a, b, False, True))
    assert int(buf[0]) == 0 and int(buf[-2:].abs().max()) == 0


def test_bmm_reference_call_site_shape(device):
    # cuda_kernels.cu:1381: col (m = n*ho*wo rows, kdim = r*s*c) x packed filter (ncol x kdim)
    n, ho, wo, c, r, s, kout = 2, 14, 14, 64, 3, 3, 128
    rng = np.random.default_rng(5)
    col = rng.integers(-255, 255, size=(1, n * ho * wo, r * s * c), endpoint=True).astype(np.int32)
    wg = rng.integers(-31, 31, size=(1, kout, r * s * c), endpoint=True).astype(np.int32)
    np.testing.assert_array_equal(_run(device, col, wg, False, True), oracle.bmm_i32(col, wg, False, True))


def test_bmm_on_a_side_stream_and_2d(device):
    a, b = _operands(31, 1, 100, 60, 77, True, False)
    s = torch.cuda.Stream()
    ad, bd = torch.from_numpy(a[0]).to(device), torch.from_numpy(b[0]).to(device)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        c = M.bmm_i32(ad, bd, trans_a=True)
    s.synchronize()
    assert tuple(c.shape) == (100, 60)
    np.testing.assert_array_equal(c.cpu().numpy(), oracle.bmm_i32(a, b, True, False)[0])
