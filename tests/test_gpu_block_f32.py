"""The blocked (locally connected) fp32 convolution on the GPU - launch_block_fprop_nhwc,
launch_block_bprop_nhwc, launch_block_grad_nhwc (cuda_kernels.cu:939-1136) through
miq_block_{fprop,bprop,grad}_nhwc_f32 - against the oracle's restatements of the reference's
cpu_block_fprop_nhwc / cpu_block_bprop_nhwc / cpu_block_grad_nhwc (cpu_ref.cpp:232-369, pinned
to the reference's own compiled functions by the CPU suite):

  - the direct kernels bit for bit (the reference loop orders and rounding), with bias in both
    modes;
  - the MFMA kernels (AUTO) within the reference's own check, verify_tensors abs 1e-4 / rel
    1e-3 (main.cpp:306-316, :394-397), on the reference's blocked suite shapes
    (main.cpp:176-186, batch cut so the oracle finishes in seconds) and edge shapes;
  - the MFMA kernels bit for bit on small-integer inputs, where every partial sum is an exact
    fp32 integer in any order, so a wrong block, tap or pixel cannot hide in rounding;
  - the bias gradient bit for bit against the oracle's restatement of its fixed order (the
    all-positions sum of launch_block_grad_nhwc), both modes, every algo;
  - a 1 x 1 block grid gives the dense entry points' bits."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle

pytestmark = pytest.mark.gpu

# name, n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups), by, bx
SUITE = [
    ("blocked_resnet_56x56_b2x2", 1, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), 2, 2),
    ("blocked_resnet_56x56_b4x4", 1, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), 4, 4),
    ("blocked_resnet_28x28_b2x4", 1, 28, 28, 128, 256, 3, 3, (1, 1, 1, 1, 1, 1, 1), 2, 4),
    ("blocked_grouped_g4_b2x2", 1, 56, 56, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 4), 2, 2),
    ("blocked_pointwise_1x1_b4x4", 1, 56, 56, 128, 256, 1, 1, (0, 0, 1, 1, 1, 1, 1), 4, 4),
    ("blocked_dilated_3x3_b2x2", 1, 64, 64, 64, 64, 3, 3, (2, 2, 1, 1, 2, 2, 1), 2, 2),
    ("blocked_small_batch_b4x4", 1, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), 4, 4),
]
EDGE = [
    ("stride2_bprop_direct", 2, 14, 12, 16, 32, 3, 3, (1, 1, 2, 2, 1, 1, 1), 7, 2),
    ("no_pad_h_gt_ho", 2, 16, 18, 8, 24, 3, 3, (0, 0, 1, 1, 1, 1, 1), 7, 4),       # bprop regions != blocks
    ("pad_wider_than_reach", 1, 9, 10, 8, 12, 1, 1, (1, 2, 1, 1, 1, 1, 1), 11, 7),  # ho > h: empty regions
    ("cg2_direct_only", 2, 10, 10, 4, 8, 3, 3, (1, 1, 1, 1, 1, 1, 2), 2, 5),      # c/groups % 4 != 0
    ("k_odd_scalar_store", 1, 12, 12, 8, 30, 3, 3, (1, 1, 1, 1, 1, 1, 1), 3, 2),
    ("5x5_dil2_b3x3", 1, 18, 18, 16, 40, 5, 5, (4, 4, 1, 1, 2, 2, 1), 3, 3),
    ("tiny_blocks_1x1_each", 2, 8, 8, 8, 16, 3, 3, (1, 1, 1, 1, 1, 1, 1), 8, 8),
    ("kg_gt_64_tiles", 1, 10, 12, 32, 136, 3, 3, (1, 1, 1, 1, 1, 1, 1), 2, 3),
]
CASES = SUITE + EDGE
IDS = [c[0] for c in CASES]


def _data(case, seed, integer=False):
    _, n, h, w, c, k, r, s, conv, by, bx = case
    rng = np.random.default_rng(seed)
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)

    def gen(shape):
        if integer:
            return rng.integers(-3, 4, size=shape).astype(np.float32)
        return rng.uniform(-1, 1, size=shape).astype(np.float32)

    return (gen((n, h, w, c)), gen((k, by, bx, r, s, c // conv[6])), gen((k * by * bx,)), gen((n, ho, wo, k)))


def _params(case):
    ph, pw, sh, sw, dh, dw, g = case[8]
    return M.BlockConv2DParams(M.Conv2DParams(ph, pw, sh, sw, dh, dw, g), case[9], case[10])


def _dims(case):
    return case[1:8]


def fprop(device, case, x, wt, bias=None, mode=0, algo="auto"):
    n, h, w, c, k, r, s = _dims(case)
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, case[8])
    y = torch.full((n, ho, wo, k), 7.0, dtype=torch.float32, device=device)
    b = None if bias is None else torch.from_numpy(bias).to(device)
    M.launch_block_fprop_nhwc(torch.from_numpy(x).to(device), torch.from_numpy(wt).to(device), y, n, h, w, c, r, s, k,
                              _params(case), b, mode, algo)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def bprop(device, case, dy, wt, algo="auto"):
    n, h, w, c, k, r, s = _dims(case)
    dx = torch.full((n, h, w, c), 7.0, dtype=torch.float32, device=device)
    M.launch_block_bprop_nhwc(torch.from_numpy(dy).to(device), torch.from_numpy(wt).to(device), dx, n, h, w, c, r, s, k,
                              _params(case), algo)
    torch.cuda.synchronize()
    return dx.cpu().numpy()


def grad(device, case, x, dy, wshape, with_dbias=False, mode=0, algo="auto"):
    n, h, w, c, k, r, s = _dims(case)
    dw = torch.full(wshape, 7.0, dtype=torch.float32, device=device)
    db = torch.full((k * case[9] * case[10],), 7.0, dtype=torch.float32, device=device) if with_dbias else None
    M.launch_block_grad_nhwc(torch.from_numpy(x).to(device), torch.from_numpy(dy).to(device), dw, n, h, w, c, r, s, k,
                             _params(case), db, mode, algo)
    torch.cuda.synchronize()
    return dw.cpu().numpy(), (None if db is None else db.cpu().numpy())


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _verify(want, got, what):
    assert oracle.verify_tensors(want, got, 1e-4, 1e-3), f"{what}: max abs err {float(np.abs(got - want).max())}"


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_block_fprop(device, case):
    x, wt, bias, _ = _data(case, 100 + CASES.index(case))
    conv = case[8]
    want = oracle.block_conv_f32(x, wt, conv)
    np.testing.assert_array_equal(_bits(fprop(device, case, x, wt, algo="direct")), _bits(want))
    _verify(want, fprop(device, case, x, wt), f"{case[0]} fprop auto")
    for mode in (0, 1):
        want_b = oracle.block_conv_f32(x, wt, conv, bias, mode)
        np.testing.assert_array_equal(_bits(fprop(device, case, x, wt, bias, mode, "direct")), _bits(want_b),
                                      err_msg=f"bias mode {mode}")
        _verify(want_b, fprop(device, case, x, wt, bias, mode), f"{case[0]} fprop+bias{mode} auto")


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_block_bprop(device, case):
    x, wt, _, dy = _data(case, 200 + CASES.index(case))
    want = oracle.block_bprop_f32(dy, wt, x.shape, case[8])
    np.testing.assert_array_equal(_bits(bprop(device, case, dy, wt, "direct")), _bits(want))
    _verify(want, bprop(device, case, dy, wt), f"{case[0]} bprop auto")


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_block_grad_and_dbias(device, case):
    x, wt, _, dy = _data(case, 300 + CASES.index(case))
    conv, by, bx = case[8], case[9], case[10]
    want = oracle.block_grad_f32(x, dy, wt.shape, conv)
    dw, _ = grad(device, case, x, dy, wt.shape, algo="direct")
    np.testing.assert_array_equal(_bits(dw), _bits(want))
    for mode in (0, 1):
        want_db = oracle.block_dbias_f32(dy, by, bx, mode)
        for algo in ("auto", "direct", "atomic"):
            dw, db = grad(device, case, x, dy, wt.shape, True, mode, algo)
            np.testing.assert_array_equal(_bits(db), _bits(want_db), err_msg=f"dbias mode {mode} algo {algo}")
            if algo != "direct":
                _verify(want, dw, f"{case[0]} grad {algo}")


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_block_mfma_exact_on_integers(device, case):
    """Small-integer inputs: every partial sum is an integer far below 2^24, exact in fp32 in any
    order, so the MFMA kernels must equal the reference loop bit for bit."""
    x, wt, bias, dy = _data(case, 400 + CASES.index(case), integer=True)
    conv = case[8]
    np.testing.assert_array_equal(_bits(fprop(device, case, x, wt, bias, 0)),
                                  _bits(oracle.block_conv_f32(x, wt, conv, bias, 0)), err_msg="fprop")
    np.testing.assert_array_equal(_bits(bprop(device, case, dy, wt)),
                                  _bits(oracle.block_bprop_f32(dy, wt, x.shape, conv)), err_msg="bprop")
    want = oracle.block_grad_f32(x, dy, wt.shape, conv)
    assert np.abs(want).max() < 2 ** 24
    for algo in ("auto", "atomic"):
        dw, _ = grad(device, case, x, dy, wt.shape, algo=algo)
        np.testing.assert_array_equal(_bits(dw), _bits(want), err_msg=f"grad {algo}")


def test_block_plan_and_dispatch(device):
    case = SUITE[0]
    n, h, w, c, k, r, s = _dims(case)
    p = _params(case)
    assert M.plan_block_f32("fprop", n, h, w, c, r, s, k, p) == "igemm"
    assert M.plan_block_f32("bprop", n, h, w, c, r, s, k, p) == "bprop_igemm"
    assert M.plan_block_f32("grad", n, h, w, c, r, s, k, p) == "grad_igemm"
    e = EDGE[0]  # stride 2: dx has no MFMA form
    assert M.plan_block_f32("bprop", *_dims(e)[:4], e[6], e[7], e[5], _params(e)) == "direct"
    with pytest.raises(M.MiqError, match="stride 1"):
        x, wt, _, dy = _data(e, 1)
        bprop(device, e, dy, wt, "igemm")
    d = EDGE[3]  # c/groups == 2: direct only
    assert M.plan_block_f32("fprop", *_dims(d)[:4], d[6], d[7], d[5], _params(d)) == "direct"
    with pytest.raises(M.MiqError, match="bias_mode"):
        x, wt, bias, _ = _data(case, 2)
        fprop(device, case, x, wt, bias, 2)


@pytest.mark.parametrize("case", [SUITE[0], EDGE[1], EDGE[4]], ids=lambda c: c[0])
def test_one_block_grid_is_the_dense_path(device, case):
    one = case[:9] + (1, 1)
    x, wt, _, dy = _data(one, 500)
    n, h, w, c, k, r, s = _dims(one)
    conv = one[8]
    dense_w = np.ascontiguousarray(wt[:, 0, 0])
    xd, wd, dyd = (torch.from_numpy(a).to(device) for a in (x, dense_w, dy))
    y = torch.empty_like(torch.from_numpy(oracle.conv_f32(x, dense_w, conv))).to(device)
    M.launch_fprop_nhwc(xd, wd, y, n, h, w, c, r, s, k, conv)
    dx = torch.empty(x.shape, dtype=torch.float32, device=device)
    M.launch_bprop_nhwc(dyd, wd, dx, n, h, w, c, r, s, k, conv)
    dw = torch.empty(dense_w.shape, dtype=torch.float32, device=device)
    M.launch_grad_nhwc(xd, dyd, dw, n, h, w, c, r, s, k, conv)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(fprop(device, one, x, wt)), _bits(y.cpu().numpy()))
    np.testing.assert_array_equal(_bits(bprop(device, one, dy, wt)), _bits(dx.cpu().numpy()))
    np.testing.assert_array_equal(_bits(grad(device, one, x, dy, wt.shape)[0][:, 0, 0]), _bits(dw.cpu().numpy()))


def test_block_grad_auto_is_deterministic(device):
    case = ("n4_b2x2", 4, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1), 2, 2)
    x, wt, _, dy = _data(case, 600)
    a = grad(device, case, x, dy, wt.shape, True, 0)
    b = grad(device, case, x, dy, wt.shape, True, 0)
    np.testing.assert_array_equal(_bits(a[0]), _bits(b[0]))
    np.testing.assert_array_equal(_bits(a[1]), _bits(b[1]))
    _verify(oracle.block_grad_f32(x, dy, wt.shape, case[8]), a[0], "grad auto n4")
