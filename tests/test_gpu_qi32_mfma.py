"""The float-code int32-accumulator convolution (launch_fprop_nhwc_qi32, the reference's own
API) on its MFMA implicit GEMM (digits of the centred codes, exact int32 wrap-around) against
the oracle's orc_conv_qi32, which the reference's cpu_fprop_nhwc_qi32 pins bit for bit:
U8 and S5 parameter layouts, per-sample zero points, fractional codes (truncation), codes far
outside 8 bits (every digit used, sums wrapping past 2^31), groups, stride, dilation,
padding, partial tiles, and c/groups % 4 != 0 (the value-by-value gather, as for the 3-channel
stem).  Integer results bit-exact."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from tests.test_gpu_parity import dev, qparams_dev

pytestmark = pytest.mark.gpu

# kind, n, h, w, c, k, r, s, conv7, code range
CASES = [
    ("u8", 2, 14, 14, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255)),
    ("s5", 3, 9, 11, 32, 48, 3, 3, (1, 1, 2, 2, 1, 1, 1), (-16, 15)),
    ("u8", 1, 12, 10, 16, 24, 3, 3, (2, 2, 1, 1, 2, 2, 2), (0, 255)),
    ("u8", 2, 8, 8, 8, 130, 1, 1, (0, 0, 1, 1, 1, 1, 1), (0, 255)),
    ("s5", 1, 20, 17, 4, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1), (-16, 15)),
    ("u8", 1, 6, 7, 12, 20, 5, 3, (4, 2, 1, 1, 1, 1, 1), (-3000, 70000)),      # wide codes
    ("u8", 2, 10, 10, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (-2.0e8, 2.0e8)),   # wrap-around sums
    ("u8", 1, 9, 9, 6, 8, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255)),              # c % 4 != 0: value-by-value gather
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}_c{c[4]}k{c[5]}r{c[6]}g{c[8][6]}" for c in CASES])
def test_qi32_float_codes_bit_exact(device, case):
    kind, n, h, w, c, k, r, s, conv, (lo, hi) = case
    rng = np.random.default_rng(4000 + CASES.index(case))
    g = conv[6]
    x = rng.uniform(lo, hi, size=(n, h, w, c)).astype(np.float32)      # fractional codes: truncated
    wt = rng.uniform(lo, hi, size=(k, r, s, c // g)).astype(np.float32)
    zlo, zhi = (0, 255) if kind == "u8" else (-128, 127)
    zp = rng.integers(zlo, zhi, size=n, endpoint=True).astype(np.int32)
    fzp = int(rng.integers(zlo, zhi, endpoint=True))
    want = oracle.conv_qi32(x, wt, conv, zp, fzp)
    tin, in_qp = qparams_dev(kind, zp, device)
    _, f_qp = qparams_dev(kind, [fzp], device)
    y = torch.full(want.shape, -7, dtype=torch.int32, device=device)
    M.launch_fprop_nhwc_qi32(tin, dev(x, device), dev(wt, device), y, n, h, w, c, r, s, k, M.Conv2DParams(*conv),
                             in_qp, f_qp)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), want)


BLOCKED = [  # kind, n, h, w, c, k, r, s, conv7, (by, bx)
    ("u8", 2, 12, 12, 16, 32, 3, 3, (1, 1, 1, 1, 1, 1, 1), (2, 2)),
    ("s5", 1, 16, 16, 32, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (4, 4)),
    ("u8", 2, 14, 10, 8, 24, 3, 3, (1, 1, 1, 1, 1, 1, 2), (2, 5)),
    ("u8", 1, 12, 12, 64, 96, 1, 1, (0, 0, 2, 2, 1, 1, 1), (3, 2)),
    ("s5", 3, 9, 8, 4, 20, 3, 3, (1, 1, 1, 1, 1, 1, 1), (1, 4)),
    ("u8", 2, 16, 16, 3, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1), (2, 2)),   # 3 channels, blocked
]


@pytest.mark.parametrize("case", BLOCKED, ids=[f"{c[0]}_b{c[9][0]}x{c[9][1]}_c{c[4]}g{c[8][6]}" for c in BLOCKED])
def test_qi32_blocked_filters_bit_exact(device, case):
    kind, n, h, w, c, k, r, s, conv, (by, bx) = case
    rng = np.random.default_rng(4500 + BLOCKED.index(case))
    g = conv[6]
    lo, hi = (0, 255) if kind == "u8" else (-16, 15)
    x = rng.uniform(lo, hi, size=(n, h, w, c)).astype(np.float32)
    wt = rng.uniform(lo, hi, size=(k, by, bx, r, s, c // g)).astype(np.float32)
    zlo, zhi = (0, 255) if kind == "u8" else (-128, 127)
    zp = rng.integers(zlo, zhi, size=n, endpoint=True).astype(np.int32)
    fzp = int(rng.integers(zlo, zhi, endpoint=True))
    want = oracle.conv_qi32(x, wt, conv, zp, fzp, (by, bx))
    tin, in_qp = qparams_dev(kind, zp, device)
    _, f_qp = qparams_dev(kind, [fzp], device)
    y = torch.full(want.shape, -7, dtype=torch.int32, device=device)
    bp = M.BlockConv2DParams(M.Conv2DParams(*conv), by, bx)
    M.launch_block_fprop_nhwc_qi32(tin, dev(x, device), dev(wt, device), y, n, h, w, c, r, s, k, bp, in_qp, f_qp)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), want)
