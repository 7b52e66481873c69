"""The float-code int32-accumulator convolution (launch_fprop_nhwc_qi32, the reference's own
API) on its stream route: a prepass writes a padded offset-int8 image and int8 filter, the
int8 stream kernel adds the offset corrections (filter row sums, per-image zero-point terms and
the pixel window sums it accumulates from its own fragments), and a final pass recomputes
everything directly only when a code left int8.  Checked against the oracle's orc_conv_qi32,
which the reference's cpu_fprop_nhwc_qi32 pins bit for bit: U8 and S5 parameter layouts with
per-sample zero points at and inside their ranges, fractional codes, strides, dilation,
padding wider than the filter reach, groups, 1x1 and 5x5 filters, codes outside int8 in one
image, in the filter or everywhere (sums wrapping past 2^31).  At the full C4 size the route
equals the implicit GEMM the float-code tests pin."""
import numpy as np
import pytest

import my_own_cnn_amd as M
import oracle
from tests.test_gpu_qi32_band import make_case, run_band

pytestmark = pytest.mark.gpu

# kind, n, h, w, c, k, r, s, conv7 (ph, pw, sh, sw, dh, dw, groups), code range
CASES = [
    ("u8", 2, 14, 14, 128, 256, 3, 3, (1, 1, 2, 2, 1, 1, 1), (0, 255)),      # C4 shape, small
    ("s5", 3, 11, 9, 64, 128, 3, 3, (1, 1, 2, 2, 1, 1, 1), (-16, 15)),
    ("u8", 1, 12, 12, 64, 128, 3, 3, (2, 2, 1, 1, 2, 2, 1), (0, 255)),       # dilation 2
    ("u8", 2, 10, 10, 128, 256, 3, 3, (1, 1, 2, 2, 1, 1, 2), (0, 255)),      # groups 2
    ("u8", 2, 9, 9, 64, 128, 1, 1, (0, 0, 2, 2, 1, 1, 1), (0, 255)),         # 1x1 stride 2
    ("s5", 1, 13, 13, 64, 128, 5, 5, (2, 2, 2, 2, 1, 1, 1), (-16, 15)),      # 5x5
    ("u8", 1, 6, 7, 64, 128, 3, 3, (3, 2, 2, 1, 1, 1, 1), (0, 255)),         # padding past the reach, stride_h only
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}_c{c[4]}k{c[5]}r{c[6]}s{c[8][2]}g{c[8][6]}" for c in CASES])
def test_qi32_route_bit_exact(device, case):
    kind, n, h, w, c, k, r, s, conv, _ = case
    x, wt, zp, fzp = make_case(case, 7000 + CASES.index(case))
    print(f"qi32 route case {case}", flush=True)
    want = oracle.conv_qi32(x, wt, conv, zp, fzp)
    np.testing.assert_array_equal(run_band(kind, x, wt, conv, zp, fzp, device, "stream"), want)


def test_qi32_route_is_auto_for_strided_shapes():
    assert M.plan_qi32(32, 56, 56, 128, 3, 3, 256, M.Conv2DParams(1, 1, 2, 2, 1, 1, 1)) == "stream"
    assert M.plan_qi32(2, 14, 14, 128, 3, 3, 256, M.Conv2DParams(1, 1, 2, 2, 1, 1, 1)) == "stream"


def test_qi32_route_extreme_zero_points(device):
    conv = (1, 1, 2, 2, 1, 1, 1)
    for kind, zps, fzp, (lo, hi) in (("u8", [0, 255], 255, (0, 255)), ("u8", [255, 0], 0, (0, 255)),
                                     ("s5", [-128, 127], 127, (-16, 15)), ("s5", [127, -128], -128, (-16, 15))):
        rng = np.random.default_rng(7100)
        x = rng.uniform(lo, hi, size=(2, 9, 9, 64)).astype(np.float32)
        wt = rng.uniform(lo, hi, size=(128, 3, 3, 64)).astype(np.float32)
        zp = np.array(zps, np.int32)
        want = oracle.conv_qi32(x, wt, conv, zp, fzp)
        np.testing.assert_array_equal(run_band(kind, x, wt, conv, zp, fzp, device, "stream"), want)


@pytest.mark.parametrize("where", ["image1", "filter", "all"])
def test_qi32_route_codes_outside_int8(device, where):
    """Any code the offset does not bring into int8 sends the call to the exact direct pass."""
    conv = (1, 1, 2, 2, 1, 1, 1)
    rng = np.random.default_rng(7200)
    x = rng.uniform(0, 255, size=(3, 10, 10, 64)).astype(np.float32)
    wt = rng.uniform(0, 255, size=(128, 3, 3, 64)).astype(np.float32)
    if where == "image1":
        x[1, 4, 5, 7] = 300.0
    elif where == "filter":
        wt[5, 1, 1, 3] = -1.0
    else:
        x = rng.uniform(-2.0e8, 2.0e8, size=x.shape).astype(np.float32)
        wt = rng.uniform(-2.0e8, 2.0e8, size=wt.shape).astype(np.float32)
    zp = np.array([3, 250, 128], np.int32)
    want = oracle.conv_qi32(x, wt, conv, zp, 17)
    np.testing.assert_array_equal(run_band("u8", x, wt, conv, zp, 17, device, "stream"), want)


def test_qi32_route_full_c4_equals_igemm(device):
    """C4 (strided downsample: N=32, 56x56, 128 -> 256, stride 2) at full size, U8 and S5 codes:
    the route equals the implicit GEMM; image 0 against the oracle as well."""
    conv = (1, 1, 2, 2, 1, 1, 1)
    for kind, rng_codes in (("u8", (0, 255)), ("s5", (-16, 15))):
        x, wt, zp, fzp = make_case((kind, 32, 56, 56, 128, 256, 3, 3, conv, rng_codes), 7300)
        a = run_band(kind, x, wt, conv, zp, fzp, device, "stream")
        b = run_band(kind, x, wt, conv, zp, fzp, device, "igemm")
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(a[:1], oracle.conv_qi32(x[:1], wt, conv, zp[:1], fzp))
