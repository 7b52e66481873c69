"""The fp32 convolution on the GPU (launch_fprop_nhwc / miq_fprop_nhwc_f32) against the
oracle's restatement of the reference's cpu_fprop_nhwc (cpu_ref.cpp:116-146):
  - the MFMA implicit GEMM within the reference's own check, verify_tensors with abs 1e-4 /
    rel 1e-3 (main.cpp:306-316), on the reference's conv_bench suite shapes (main.cpp:163-174,
    batch cut to keep the oracle in seconds) and on edge shapes: channel tiles and pixel
    tiles partly filled, taps spanning a chunk (c/groups = 4, 12), stride 3, padding wider
    than the filter, 5x5 and 7x7 taps, K % 4 != 0 (scalar stores), an unaligned output;
  - the direct kernel bit for bit (it keeps the reference loop's order and rounding)."""
import numpy as np
import pytest
import torch

import my_own_cnn_amd as M
import oracle

pytestmark = pytest.mark.gpu

# name, n, h, w, c, k, r, s, (ph, pw, sh, sw, dh, dw, groups)
SUITE = [
    ("resnet_like_56x56", 1, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("resnet_like_28x28", 1, 28, 28, 128, 256, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("downsample_stride2", 1, 112, 112, 32, 32, 3, 3, (1, 1, 2, 2, 1, 1, 1)),
    ("depthwise_3x3", 1, 56, 56, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 128)),
    ("grouped_g4", 1, 56, 56, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 4)),
    ("pointwise_1x1", 1, 56, 56, 128, 256, 1, 1, (0, 0, 1, 1, 1, 1, 1)),
    ("dilated_3x3", 1, 64, 64, 64, 64, 3, 3, (2, 2, 1, 1, 2, 2, 1)),
    ("small_batch", 1, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
]
EDGE = [
    ("kg24_m_tail", 2, 9, 13, 16, 24, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("cg4_taps_span", 1, 17, 19, 4, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("cg12_taps_span", 2, 11, 7, 24, 36, 3, 3, (1, 1, 2, 1, 1, 1, 2)),
    ("stride3_wide_pad", 1, 15, 21, 32, 96, 3, 3, (4, 3, 3, 3, 1, 1, 1)),
    ("5x5_dil2", 1, 20, 20, 16, 80, 5, 5, (4, 4, 1, 1, 2, 2, 1)),
    ("7x7_s2_c4", 2, 30, 30, 4, 64, 7, 7, (3, 3, 2, 2, 1, 1, 1)),
    ("k_odd_scalar_store", 1, 10, 10, 8, 30, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("groups3_kg5", 1, 8, 9, 12, 15, 1, 3, (0, 1, 1, 1, 1, 1, 3)),
    ("depthwise_s2_d2", 2, 15, 13, 36, 36, 3, 5, (2, 3, 2, 1, 2, 1, 36)),
]
CASES = SUITE + EDGE


def _data(case, seed):
    _, n, h, w, c, k, r, s, conv = case
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, size=(n, h, w, c)).astype(np.float32)
    wt = rng.uniform(-1, 1, size=(k, r, s, c // conv[6])).astype(np.float32)
    return x, wt


def _run(device, x, wt, conv, algo):
    ph, pw, sh, sw, dh, dw, g = conv
    xd, wd = torch.from_numpy(x).to(device), torch.from_numpy(wt).to(device)
    y = M.conv2d_nhwc_f32(xd, wd, stride=(sh, sw), padding=(ph, pw), dilation=(dh, dw), groups=g, algo=algo)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fp32_conv_matches_reference_cpu(device, case):
    x, wt = _data(case, 500 + CASES.index(case))
    conv = case[8]
    want = oracle.conv_f32(x, wt, conv)
    got = _run(device, x, wt, conv, "auto")
    assert oracle.verify_tensors(want, got, 1e-4, 1e-3), float(np.abs(got - want).max())
    if conv[6] == case[4] == case[5]:  # depthwise: AUTO's 4-channel kernel keeps the reference order
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    direct = _run(device, x, wt, conv, "direct")
    np.testing.assert_array_equal(direct.view(np.uint32), want.view(np.uint32))


def test_fp32_igemm_is_what_auto_runs_where_it_applies(device):
    x, wt = _data(SUITE[0], 1)
    conv = SUITE[0][8]
    a = _run(device, x, wt, conv, "auto")
    b = _run(device, x, wt, conv, "igemm")
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    with pytest.raises(M.MiqError, match="% 4"):
        _run(device, *_data(SUITE[3], 2)[:2], SUITE[3][8], "igemm")  # depthwise: c/groups == 1


def test_fp32_unaligned_output_and_empty_image(device):
    x, wt = _data(EDGE[0], 3)
    conv = EDGE[0][8]
    n, h, w, c = x.shape
    k = wt.shape[0]
    want = oracle.conv_f32(x, wt, conv)
    buf = torch.zeros(want.size + 1, dtype=torch.float32, device=device)
    xd, wd = torch.from_numpy(x).to(device), torch.from_numpy(wt).to(device)
    M.launch_fprop_nhwc(xd, wd, buf[1:], n, h, w, c, 3, 3, k, conv, algo="igemm")
    torch.cuda.synchronize()
    got = buf[1:].cpu().numpy().reshape(want.shape)
    assert oracle.verify_tensors(want, got) and float(buf[0]) == 0.0
    # H == 0 with padding: every tap is outside the image, the output is zeros
    xe = torch.empty((1, 0, 4, 8), dtype=torch.float32, device=device)
    we = torch.ones((8, 1, 1, 8), dtype=torch.float32, device=device)
    ye = M.conv2d_nhwc_f32(xe, we, padding=1)
    torch.cuda.synchronize()
    assert tuple(ye.shape) == (1, 2, 6, 8) and float(ye.abs().max()) == 0.0


BACKWARD = [c for c in CASES if c[0] not in ("resnet_like_28x28", "downsample_stride2", "pointwise_1x1")] + [
    ("resnet_like_28x28_n1_small", 1, 14, 14, 128, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("downsample_stride2_small", 1, 40, 40, 32, 32, 3, 3, (1, 1, 2, 2, 1, 1, 1)),
]


@pytest.mark.parametrize("case", BACKWARD, ids=[c[0] for c in BACKWARD])
def test_fp32_bprop_and_grad_bit_exact(device, case):
    _, n, h, w, c, k, r, s, conv = case
    x, wt = _data(case, 700 + BACKWARD.index(case))
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    dy = np.random.default_rng(800 + BACKWARD.index(case)).uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)
    xd, wd, dyd = (torch.from_numpy(a).to(device) for a in (x, wt, dy))
    dx = torch.full(x.shape, 7.0, dtype=torch.float32, device=device)
    dw = torch.full(wt.shape, 7.0, dtype=torch.float32, device=device)
    M.launch_bprop_nhwc(dyd, wd, dx, n, h, w, c, r, s, k, conv, algo="direct")
    M.launch_grad_nhwc(xd, dyd, dw, n, h, w, c, r, s, k, conv, algo="direct")
    torch.cuda.synchronize()
    want_dx = oracle.bprop_f32(dy, wt, x.shape, conv)
    np.testing.assert_array_equal(dx.cpu().numpy().view(np.uint32), want_dx.view(np.uint32))
    np.testing.assert_array_equal(dw.cpu().numpy().view(np.uint32), oracle.grad_f32(x, dy, wt.shape, conv).view(np.uint32))
    # AUTO: the MFMA implicit GEMM over dy with the flipped filter where it applies (stride 1,
    # (k/groups) % 4 == 0), checked with the reference's verify rule
    dx.fill_(7.0)
    M.launch_bprop_nhwc(dyd, wd, dx, n, h, w, c, r, s, k, conv)
    torch.cuda.synchronize()
    got = dx.cpu().numpy()
    assert oracle.verify_tensors(want_dx, got, 1e-4, 1e-3), float(np.abs(got - want_dx).max())
    # AUTO grad: the MFMA GEMM over pixels, split over workgroups (atomics), verify rule
    dw.fill_(7.0)
    M.launch_grad_nhwc(xd, dyd, dw, n, h, w, c, r, s, k, conv)
    torch.cuda.synchronize()
    want_dw = oracle.grad_f32(x, dy, wt.shape, conv)
    got = dw.cpu().numpy()
    assert oracle.verify_tensors(want_dw, got, 1e-4, 1e-3), float(np.abs(got - want_dw).max())


DW_BPROP = [
    ("dw_s1", 2, 13, 11, 24, 24, 3, 3, (1, 1, 1, 1, 1, 1, 24)),
    ("dw_s2_d2", 2, 15, 13, 36, 36, 3, 5, (2, 3, 2, 1, 2, 1, 36)),
    ("dw_s3_pad0", 1, 17, 16, 8, 8, 5, 3, (0, 1, 3, 2, 1, 1, 8)),
]


@pytest.mark.parametrize("case", DW_BPROP, ids=[c[0] for c in DW_BPROP])
def test_fp32_depthwise_bprop_bit_exact(device, case):
    # AUTO's depthwise dx kernel keeps cpu_bprop_nhwc's tap order: bit-exact at any stride
    _, n, h, w, c, k, r, s, conv = case
    x, wt = _data(case, 900 + DW_BPROP.index(case))
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    dy = np.random.default_rng(950 + DW_BPROP.index(case)).uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)
    p = M.Conv2DParams(*conv)
    assert M.plan_f32("bprop", n, h, w, c, r, s, k, p) == "depthwise"
    wd, dyd = torch.from_numpy(wt).to(device), torch.from_numpy(dy).to(device)
    dx = torch.full(x.shape, 7.0, dtype=torch.float32, device=device)
    M.launch_bprop_nhwc(dyd, wd, dx, n, h, w, c, r, s, k, conv)
    torch.cuda.synchronize()
    want = oracle.bprop_f32(dy, wt, x.shape, conv)
    np.testing.assert_array_equal(dx.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_fp32_direct_bprop_four_channels_and_unaligned(device):
    # (c/groups) % 4 == 0 with aligned dx and filter: 4 channels per thread; an unaligned dx takes
    # the one-element kernel; both give cpu_bprop_nhwc's bits (stride 2, groups 2, K not a multiple of 4)
    case = ("s2_g2", 2, 19, 17, 16, 18, 3, 3, (1, 1, 2, 2, 1, 1, 2))
    _, n, h, w, c, k, r, s, conv = case
    x, wt = _data(case, 990)
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    dy = np.random.default_rng(991).uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)
    want = oracle.bprop_f32(dy, wt, x.shape, conv)
    wd, dyd = torch.from_numpy(wt).to(device), torch.from_numpy(dy).to(device)
    dx = torch.full(x.shape, 7.0, dtype=torch.float32, device=device)
    M.launch_bprop_nhwc(dyd, wd, dx, n, h, w, c, r, s, k, conv, algo="direct")
    buf = torch.full((x.size + 1,), 7.0, dtype=torch.float32, device=device)
    M.launch_bprop_nhwc(dyd, wd, buf[1:], n, h, w, c, r, s, k, conv, algo="direct")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dx.cpu().numpy().view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(buf[1:].cpu().numpy().reshape(want.shape).view(np.uint32), want.view(np.uint32))
    assert float(buf[0]) == 7.0


def test_fp32_bprop_igemm_applies_at_stride_1_only(device):
    x, wt = _data(SUITE[0], 9)
    conv = SUITE[0][8]
    n, h, w, c = x.shape
    k, r, s = wt.shape[:3]
    dy = torch.rand((n, h, w, k), device=device) * 2 - 1
    dx = torch.empty((n, h, w, c), device=device)
    wd = torch.from_numpy(wt).to(device)
    M.launch_bprop_nhwc(dy, wd, dx, n, h, w, c, r, s, k, conv, algo="igemm")
    torch.cuda.synchronize()
    assert oracle.verify_tensors(oracle.bprop_f32(dy.cpu().numpy(), wt, x.shape, conv), dx.cpu().numpy())
    with pytest.raises(M.MiqError, match="stride 1"):
        M.launch_bprop_nhwc(dy, wd, dx, n, h, w, c, r, s, k, (1, 1, 2, 2, 1, 1, 1), algo="igemm")


# Shapes with many pixel splits (the MFMA GEMM: several column tiles; depthwise: many runs)
# so that the ordered sums add hundreds of partial tiles.
DETERMINISTIC = [
    ("igemm_56x56_n4", 4, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("igemm_grouped_g4", 2, 28, 28, 64, 32, 3, 3, (1, 1, 2, 2, 1, 1, 4)),
    ("depthwise_n4", 4, 56, 56, 128, 128, 3, 3, (1, 1, 1, 1, 1, 1, 128)),
]


@pytest.mark.parametrize("case", DETERMINISTIC, ids=[c[0] for c in DETERMINISTIC])
def test_fp32_grad_auto_is_deterministic(device, case):
    """AUTO grad adds the split partial sums in a fixed order: two calls give the same bits on
    random inputs, and so does the caller-workspace form.  Values: with small integer inputs
    every partial sum is an integer below 2^24, exact in fp32 in any order, so AUTO, the
    workspace form and the float-atomic opt-in must all equal cpu_grad_nhwc bit for bit (a
    dropped, repeated or misplaced term cannot hide in rounding)."""
    name, n, h, w, c, k, r, s, conv = case
    x, wt = _data(case, 900 + DETERMINISTIC.index(case))
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    rng = np.random.default_rng(950 + DETERMINISTIC.index(case))
    dy = rng.uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)
    nbytes = M.grad_workspace_size(n, h, w, c, r, s, k, conv)
    assert nbytes > 0, f"{name}: expected a multi-split shape"
    ws = torch.full((nbytes // 4 + 3,), float("nan"), dtype=torch.float32, device=device)

    def grad(xa, dya, **kw):
        dw = torch.full(wt.shape, 7.0, dtype=torch.float32, device=device)
        M.launch_grad_nhwc(torch.from_numpy(xa).to(device), torch.from_numpy(dya).to(device), dw, n, h, w, c, r, s, k,
                           conv, **kw)
        torch.cuda.synchronize()
        return dw.cpu().numpy()

    a, b, cws = grad(x, dy), grad(x, dy), grad(x, dy, workspace=ws)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"{name}: AUTO twice")
    np.testing.assert_array_equal(cws.view(np.uint32), a.view(np.uint32), err_msg=f"{name}: workspace form")
    with pytest.raises(M.MiqError, match="smaller"):
        grad(x, dy, workspace=ws[: nbytes // 8])
    xi = rng.integers(-3, 4, size=x.shape).astype(np.float32)
    dyi = rng.integers(-3, 4, size=dy.shape).astype(np.float32)
    want = oracle.grad_f32(xi, dyi, wt.shape, conv)
    assert np.abs(want).max() < 2 ** 24
    for kw in ({}, {"workspace": ws}, {"algo": "atomic"}):
        np.testing.assert_array_equal(grad(xi, dyi, **kw).view(np.uint32), want.view(np.uint32), err_msg=f"{name} {kw}")
