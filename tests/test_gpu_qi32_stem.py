"""The float-code int32-accumulator convolution (launch_fprop_nhwc_qi32, the reference's own
API) on its stem route, for stride-2 layers with 1 to 4 channels: a prepass writes the image as
offset-int8 rows padded to a multiple of 16 bytes (padded taps at zx - offset) and the filter
value by value, the space-to-depth stem kernel adds the offset corrections (filter row sums,
per-image zero-point terms and the pixel window sums it accumulates from its own fragments
under a mask of the filter's taps), and a final pass recomputes everything directly only when a
code left int8.  Checked against the oracle's orc_conv_qi32, which the reference's
cpu_fprop_nhwc_qi32 pins bit for bit: U8 and S5 parameter layouts, per-sample zero points at and
inside their ranges, fractional codes, 1x1 to 7x7 filters (odd, even and not square), 1 to 4
channels, padding 0 to 3 (also unequal), widths whose rows are not a multiple of 16 bytes,
two 64-channel tiles, codes outside int8 in one image, in the filter or everywhere (sums
wrapping past 2^31).  At the full C5 size the route equals the implicit GEMM."""
import numpy as np
import pytest

import my_own_cnn_amd as M
import oracle
from tests.test_gpu_qi32_band import make_case, run_band

pytestmark = pytest.mark.gpu

# kind, n, h, w, c, k, r, s, conv7 (ph, pw, sh, sw, dh, dw, groups), code range
CASES = [
    ("u8", 2, 20, 18, 3, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1), (0, 255)),       # the stem, small
    ("s5", 2, 21, 17, 3, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1), (-16, 15)),      # odd sizes, rows of 51 bytes
    ("u8", 1, 9, 16, 1, 64, 3, 3, (1, 1, 2, 2, 1, 1, 1), (0, 255)),        # one channel
    ("u8", 2, 13, 10, 2, 128, 5, 5, (2, 2, 2, 2, 1, 1, 1), (0, 255)),      # two channels, two tiles
    ("s5", 1, 10, 6, 4, 64, 4, 4, (1, 1, 2, 2, 1, 1, 1), (-16, 15)),       # even filter, four channels
    ("u8", 3, 7, 32, 3, 64, 1, 1, (0, 0, 2, 2, 1, 1, 1), (0, 255)),        # 1x1 stride 2
    ("u8", 2, 11, 24, 3, 64, 7, 7, (0, 0, 2, 2, 1, 1, 1), (0, 255)),       # no padding
    ("u8", 1, 9, 16, 3, 64, 3, 2, (3, 1, 2, 2, 1, 1, 1), (0, 255)),        # unequal filter and padding
    ("u8", 1, 224, 224, 3, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1), (0, 255)),     # one full stem image
    ("u8", 1, 12, 32, 3, 64, 5, 5, (2, 2, 2, 2, 1, 1, 1), (0, 255)),      # codes 2 past a float4 boundary
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}_n{c[1]}h{c[2]}w{c[3]}c{c[4]}k{c[5]}r{c[6]}s{c[7]}" for c in CASES])
def test_qi32_stem_route_bit_exact(device, case):
    kind, n, h, w, c, k, r, s, conv, _ = case
    x, wt, zp, fzp = make_case(case, 7500 + CASES.index(case))
    print(f"qi32 stem route case {case}", flush=True)
    want = oracle.conv_qi32(x, wt, conv, zp, fzp)
    np.testing.assert_array_equal(run_band(kind, x, wt, conv, zp, fzp, device, "stem_s2d"), want)


def test_qi32_stem_route_is_auto_for_thin_strided_shapes():
    assert M.plan_qi32(32, 224, 224, 3, 7, 7, 64, M.Conv2DParams(3, 3, 2, 2, 1, 1, 1)) == "stem_s2d"
    assert M.plan_qi32(2, 20, 18, 3, 7, 7, 64, M.Conv2DParams(3, 3, 2, 2, 1, 1, 1)) == "stem_s2d"
    # stride 1 and five channels are not its shapes
    assert M.plan_qi32(2, 20, 18, 3, 7, 7, 64, M.Conv2DParams(3, 3, 1, 1, 1, 1, 1)) != "stem_s2d"
    assert M.plan_qi32(2, 20, 18, 5, 7, 7, 64, M.Conv2DParams(3, 3, 2, 2, 1, 1, 1)) != "stem_s2d"


def test_qi32_stem_route_extreme_zero_points(device):
    conv = (3, 3, 2, 2, 1, 1, 1)
    for kind, zps, fzp, (lo, hi) in (("u8", [0, 255], 255, (0, 255)), ("u8", [255, 0], 0, (0, 255)),
                                     ("s5", [-128, 127], 127, (-16, 15)), ("s5", [127, -128], -128, (-16, 15))):
        rng = np.random.default_rng(7600)
        x = rng.uniform(lo, hi, size=(2, 15, 14, 3)).astype(np.float32)
        wt = rng.uniform(lo, hi, size=(64, 7, 7, 3)).astype(np.float32)
        zp = np.array(zps, np.int32)
        want = oracle.conv_qi32(x, wt, conv, zp, fzp)
        np.testing.assert_array_equal(run_band(kind, x, wt, conv, zp, fzp, device, "stem_s2d"), want)


@pytest.mark.parametrize("where", ["image1", "filter", "all"])
def test_qi32_stem_route_codes_outside_int8(device, where):
    """Any code the offset does not bring into int8 sends the call to the exact direct pass."""
    conv = (3, 3, 2, 2, 1, 1, 1)
    rng = np.random.default_rng(7700)
    x = rng.uniform(0, 255, size=(3, 16, 16, 3)).astype(np.float32)
    wt = rng.uniform(0, 255, size=(64, 7, 7, 3)).astype(np.float32)
    if where == "image1":
        x[1, 4, 5, 2] = 300.0
    elif where == "filter":
        wt[5, 6, 6, 2] = -1.0
    else:
        x = rng.uniform(-2.0e8, 2.0e8, size=x.shape).astype(np.float32)
        wt = rng.uniform(-2.0e8, 2.0e8, size=wt.shape).astype(np.float32)
    zp = np.array([3, 250, 128], np.int32)
    want = oracle.conv_qi32(x, wt, conv, zp, 17)
    np.testing.assert_array_equal(run_band("u8", x, wt, conv, zp, 17, device, "stem_s2d"), want)


def test_qi32_stem_route_full_c5_equals_igemm(device):
    """C5 (the ResNet stem: N=32, 224x224x3 -> 64, 7x7 stride 2, padding 3) at full size, U8 and
    S5 codes: the route equals the implicit GEMM; image 0 against the oracle as well."""
    conv = (3, 3, 2, 2, 1, 1, 1)
    for kind, rng_codes in (("u8", (0, 255)), ("s5", (-16, 15))):
        x, wt, zp, fzp = make_case((kind, 32, 224, 224, 3, 64, 7, 7, conv, rng_codes), 7800)
        a = run_band(kind, x, wt, conv, zp, fzp, device, "stem_s2d")
        b = run_band(kind, x, wt, conv, zp, fzp, device, "igemm")
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(a[:1], oracle.conv_qi32(x[:1], wt, conv, zp[:1], fzp))
