"""The float-code int32-accumulator convolution (launch_fprop_nhwc_qi32, the reference's own
API) on its row-band kernel (codes staged once per band as offset int8 values, the int8 band
kernel's MFMA loop, window and filter sums for the offsets) against the oracle's
orc_conv_qi32, which the reference's cpu_fprop_nhwc_qi32 pins bit for bit.  Covers U8 and S5
parameter layouts with per-sample zero points, fractional codes, padding, stride_h and
dilation, groups, partial and multiple 64-channel tiles, odd and even K-block counts, the
widest output row, and workgroups whose codes leave the int8 window (some or all images),
which take the kernel's direct path.  Integer results bit-exact; at the full C2 size the band
kernel equals the implicit GEMM the oracle tests pin."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle
from tests.test_gpu_parity import dev, qparams_dev

pytestmark = pytest.mark.gpu

# kind, n, h, w, c, k, r, s, conv7 (ph, pw, sh, sw, dh, dw, groups), code range
CASES = [
    ("u8", 2, 14, 14, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255)),
    ("s5", 3, 9, 11, 64, 48, 3, 3, (1, 1, 1, 1, 1, 1, 1), (-16, 15)),       # partial tile
    ("u8", 2, 7, 7, 128, 512, 1, 1, (0, 0, 1, 1, 1, 1, 1), (0, 255)),       # 8 tiles, 2 quads, even KB
    ("u8", 1, 13, 10, 64, 32, 3, 3, (2, 1, 2, 1, 2, 1, 1), (0, 255)),       # stride_h 2, dilation_h 2
    ("s5", 2, 9, 9, 128, 64, 3, 3, (1, 1, 1, 1, 1, 2, 2), (-16, 15)),       # groups 2, dilation_w 2
    ("u8", 1, 8, 64, 64, 16, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255)),        # Wo = 64, 16 channels
    ("u8", 2, 11, 9, 64, 80, 5, 1, (2, 0, 1, 1, 1, 1, 1), (0, 255)),        # 5 x 1 filter, odd KB
    ("s5", 1, 6, 12, 192, 64, 1, 3, (0, 1, 1, 1, 1, 1, 1), (-16, 15)),      # 3 quads, KB = 9
    ("u8", 2, 10, 10, 64, 64, 2, 2, (1, 1, 1, 1, 1, 1, 1), (0, 255)),       # KB = 4, asymmetric padding use
    ("u8", 1, 5, 5, 64, 128, 3, 3, (3, 3, 1, 1, 1, 1, 1), (0, 255)),        # padding wider than the filter reach
]


def run_band(kind, x, wt, conv, zp, fzp, device, algo="band"):
    n, h, w, c = x.shape
    k, r, s = wt.shape[0], wt.shape[1], wt.shape[2]
    tin, in_qp = qparams_dev(kind, zp, device)
    _, f_qp = qparams_dev(kind, [fzp], device)
    ho, wo = M.infer_conv_shape(n, h, w, c, r, s, k, M.Conv2DParams(*conv))
    y = torch.full((n, ho, wo, k), -7, dtype=torch.int32, device=device)
    M.fprop_nhwc_qi32_algo(tin, dev(x, device), dev(wt, device), y, n, h, w, c, r, s, k, M.Conv2DParams(*conv),
                           in_qp, f_qp, algo=algo)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def make_case(case, seed):
    kind, n, h, w, c, k, r, s, conv, (lo, hi) = case
    rng = np.random.default_rng(seed)
    g = conv[6]
    x = rng.uniform(lo, hi, size=(n, h, w, c)).astype(np.float32)
    wt = rng.uniform(lo, hi, size=(k, r, s, c // g)).astype(np.float32)
    zlo, zhi = (0, 255) if kind == "u8" else (-128, 127)
    zp = rng.integers(zlo, zhi, size=n, endpoint=True).astype(np.int32)
    fzp = int(rng.integers(zlo, zhi, endpoint=True))
    return x, wt, zp, fzp


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}_c{c[4]}k{c[5]}r{c[6]}s{c[7]}g{c[8][6]}" for c in CASES])
def test_qi32_band_bit_exact(device, case):
    kind, n, h, w, c, k, r, s, conv, _ = case
    assert M.plan_qi32(n, h, w, c, r, s, k, M.Conv2DParams(*conv)) == "band"
    x, wt, zp, fzp = make_case(case, 6000 + CASES.index(case))
    print(f"qi32 band case {case}", flush=True)
    want = oracle.conv_qi32(x, wt, conv, zp, fzp)
    np.testing.assert_array_equal(run_band(kind, x, wt, conv, zp, fzp, device), want)


def test_qi32_band_extreme_zero_points(device):
    """Zero points at the ends of the parameter type's range (0 and 255, -128 and 127): the
    padded-tap value zx - offset is then at the ends of int8."""
    for kind, zps, fzp, (lo, hi) in (("u8", [0, 255], 255, (0, 255)), ("u8", [255, 0], 0, (0, 255)),
                                     ("s5", [-128, 127], 127, (-16, 15)), ("s5", [127, -128], -128, (-16, 15))):
        conv = (1, 1, 1, 1, 1, 1, 1)
        rng = np.random.default_rng(6100)
        x = rng.uniform(lo, hi, size=(2, 9, 9, 64)).astype(np.float32)
        wt = rng.uniform(lo, hi, size=(64, 3, 3, 64)).astype(np.float32)
        zp = np.array(zps, np.int32)
        want = oracle.conv_qi32(x, wt, conv, zp, fzp)
        np.testing.assert_array_equal(run_band(kind, x, wt, conv, zp, fzp, device), want)


@pytest.mark.parametrize("where", ["image1", "filter", "all"])
def test_qi32_band_codes_outside_int8(device, where):
    """Codes the offset does not bring into int8: the workgroups that stage one compute their
    outputs directly; the others keep the MFMA path.  Sums wrap past 2^31."""
    conv = (1, 1, 1, 1, 1, 1, 1)
    rng = np.random.default_rng(6200)
    x = rng.uniform(0, 255, size=(3, 10, 10, 64)).astype(np.float32)
    wt = rng.uniform(0, 255, size=(64, 3, 3, 64)).astype(np.float32)
    if where == "image1":
        x[1, 4, 5, 7] = 300.0           # one code of image 1 (its bands only)
    elif where == "filter":
        wt[5, 1, 1, 3] = -1.0           # every workgroup stages the filter
    else:
        x = rng.uniform(-2.0e8, 2.0e8, size=x.shape).astype(np.float32)
        wt = rng.uniform(-2.0e8, 2.0e8, size=wt.shape).astype(np.float32)
    zp = np.array([3, 250, 128], np.int32)
    fzp = 17
    want = oracle.conv_qi32(x, wt, conv, zp, fzp)
    np.testing.assert_array_equal(run_band("u8", x, wt, conv, zp, fzp, device), want)


def test_qi32_band_full_c2_equals_igemm(device):
    """C2 (ResNet-50 3x3: N=32, 56x56, 64 -> 64) at full size, U8 and S5 codes: the band kernel
    equals the implicit GEMM (pinned to the oracle above and in the float-code tests)."""
    conv = (1, 1, 1, 1, 1, 1, 1)
    for kind, (lo, hi) in (("u8", (0, 255)), ("s5", (-16, 15))):
        x, wt, zp, fzp = make_case((kind, 32, 56, 56, 64, 64, 3, 3, conv, (lo, hi)), 6300)
        a = run_band(kind, x, wt, conv, zp, fzp, device, "band")
        b = run_band(kind, x, wt, conv, zp, fzp, device, "igemm")
        np.testing.assert_array_equal(a, b)
        # image 0 against the oracle as well
        want0 = oracle.conv_qi32(x[:1], wt, conv, zp[:1], fzp)
        np.testing.assert_array_equal(a[:1], want0)


# blocked filters [K, By, Bx, R, S, C/groups] (launch_block_fprop_nhwc_qi32) on the band route:
# kind, n, h, w, c, k, r, s, conv7, code range, (By, Bx)
BLOCK_CASES = [
    ("u8", 2, 14, 14, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255), (2, 2)),      # 7 x 7 blocks
    ("s5", 2, 16, 32, 64, 48, 3, 3, (1, 1, 1, 1, 1, 1, 1), (-16, 15), (2, 4)),     # partial tile, 8 x 8 blocks
    ("u8", 1, 9, 60, 128, 64, 1, 1, (0, 0, 1, 1, 1, 1, 1), (0, 255), (3, 3)),      # block width 20: a partial segment
    ("u8", 2, 12, 16, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 2), (0, 255), (2, 2)),    # groups 2
    ("u8", 1, 17, 24, 64, 64, 3, 3, (1, 1, 2, 1, 1, 1, 1), (0, 255), (3, 2)),      # stride_h 2 (Ho 9)
    ("s5", 1, 8, 64, 64, 32, 3, 3, (1, 1, 1, 1, 1, 1, 1), (-16, 15), (1, 1)),      # a 1 x 1 block grid
    ("u8", 2, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255), (4, 4)),      # C2's rows, 14 x 14 blocks
]


def run_block(kind, x, wt, conv, zp, fzp, block, device):
    n, h, w, c = x.shape
    k, r, s = wt.shape[0], wt.shape[3], wt.shape[4]
    tin, in_qp = qparams_dev(kind, zp, device)
    _, f_qp = qparams_dev(kind, [fzp], device)
    p = M.BlockConv2DParams(M.Conv2DParams(*conv), block[0], block[1])
    ho, wo = M.infer_conv_shape(n, h, w, c, r, s, k, M.Conv2DParams(*conv))
    y = torch.full((n, ho, wo, k), -7, dtype=torch.int32, device=device)
    M.launch_block_fprop_nhwc_qi32(tin, dev(x, device), dev(wt, device), y, n, h, w, c, r, s, k, p, in_qp, f_qp)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def make_block_case(case, seed):
    kind, n, h, w, c, k, r, s, conv, (lo, hi), block = case
    rng = np.random.default_rng(seed)
    g = conv[6]
    x = rng.uniform(lo, hi, size=(n, h, w, c)).astype(np.float32)
    wt = rng.uniform(lo, hi, size=(k, block[0], block[1], r, s, c // g)).astype(np.float32)
    zlo, zhi = (0, 255) if kind == "u8" else (-128, 127)
    zp = rng.integers(zlo, zhi, size=n, endpoint=True).astype(np.int32)
    fzp = int(rng.integers(zlo, zhi, endpoint=True))
    return x, wt, zp, fzp


@pytest.mark.parametrize("case", BLOCK_CASES,
                         ids=[f"{c[0]}_h{c[2]}w{c[3]}c{c[4]}k{c[5]}r{c[6]}g{c[8][6]}b{c[10][0]}x{c[10][1]}" for c in BLOCK_CASES])
def test_qi32_band_blocked_bit_exact(device, case):
    kind, n, h, w, c, k, r, s, conv, _, block = case
    p = M.BlockConv2DParams(M.Conv2DParams(*conv), block[0], block[1])
    assert M.plan_block_qi32(n, h, w, c, r, s, k, p) == "band"
    x, wt, zp, fzp = make_block_case(case, 6400 + BLOCK_CASES.index(case))
    print(f"qi32 blocked band case {case}", flush=True)
    want = oracle.conv_qi32(x, wt, conv, zp, fzp, block=block)
    np.testing.assert_array_equal(run_block(kind, x, wt, conv, zp, fzp, block, device), want)


def test_qi32_band_blocked_codes_outside_int8(device):
    """A code outside int8 in one image: its workgroups compute directly (with the block's
    filter), the others keep the MFMA path."""
    case = ("u8", 3, 12, 16, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), (0, 255), (2, 2))
    x, wt, zp, fzp = make_block_case(case, 6500)
    x[1, 7, 9, 5] = 300.0
    wt[3, 1, 0, 2, 1, 7] = -1.0  # every workgroup of the block stages a filter value outside int8
    want = oracle.conv_qi32(x, wt, case[8], zp, fzp, block=(2, 2))
    np.testing.assert_array_equal(run_block("u8", x, wt, case[8], zp, fzp, (2, 2), device), want)


def test_qi32_band_blocked_full_c2(device):
    """C2 with 2 x 2 and 4 x 4 filter blocks at full size (N = 32): the band route, images 0
    and 31 against the oracle."""
    conv = (1, 1, 1, 1, 1, 1, 1)
    for block in ((2, 2), (4, 4)):
        case = ("u8", 32, 56, 56, 64, 64, 3, 3, conv, (0, 255), block)
        x, wt, zp, fzp = make_block_case(case, 6600 + block[0])
        p = M.BlockConv2DParams(M.Conv2DParams(*conv), block[0], block[1])
        assert M.plan_block_qi32(32, 56, 56, 64, 3, 3, 64, p) == "band"
        print(f"qi32 blocked full C2 {block}", flush=True)
        y = run_block("u8", x, wt, conv, zp, fzp, block, device)
        for i in (0, 31):
            want = oracle.conv_qi32(x[i:i + 1], wt, conv, zp[i:i + 1], fzp, block=block)
            np.testing.assert_array_equal(y[i:i + 1], want, err_msg=f"{block} image {i}")
