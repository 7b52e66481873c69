"""Parity of the HIP library with the oracle and the reference's golden vectors, through
the C-ABI, on the GPU.  Integer results must be bit-exact; the fp32 dequantized view is
required bit-exact as well (its tolerance, 1 ulp, is met with 0 ulp)."""
import hashlib
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
import my_own_cnn_amd as M
from my_own_cnn_amd import workloads as W
from tests.golden import cases

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def qparams_dev(kind, zps, device):
    tin = M.DataType.LinQuantU8 if kind == "u8" else M.DataType.LinQuantS5
    arr = M.qparams_array(tin, list(zps), n_bins=31)
    return tin, torch.from_numpy(np.frombuffer(arr.tobytes(), np.uint8).copy()).to(device)


def run_qi32(c, device):
    x, w = c["x"], c["w"]
    n, h, wd, ch = x.shape
    k = w.shape[0]
    r, s = w.shape[-3], w.shape[-2]
    tin, in_qp = qparams_dev(c["kind"], c["zp"], device)
    _, f_qp = qparams_dev(c["kind"], [c["fzp"]], device)
    y = torch.full(c["y"].shape, -7, dtype=torch.int32, device=device)
    p = M.Conv2DParams(*c["conv"])
    if tuple(c["block"]) == (0, 0):
        M.launch_fprop_nhwc_qi32(tin, dev(x, device), dev(w, device), y, n, h, wd, ch, r, s, k, p, in_qp, f_qp)
    else:
        bp = M.BlockConv2DParams(p, *c["block"])
        M.launch_block_fprop_nhwc_qi32(tin, dev(x, device), dev(w, device), y, n, h, wd, ch, r, s, k, bp, in_qp, f_qp)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("name", ["regular_u8", "regular_s5", "blocked_u8", "blocked_s5"])
def test_quant_conv_test_cases(device, name):
    c = cases.quant_conv_test_cases()[name]
    np.testing.assert_array_equal(run_qi32(c, device), c["y"])


def test_qi32_extra_cases(device):
    for name, c in cases.qi32_cases().items():
        np.testing.assert_array_equal(run_qi32(c, device), c["y"], err_msg=name)


def test_quant_conv_test_program(device):
    exe = ROOT / "tests" / "cpp" / "bin" / "quant_conv_test"
    assert exe.exists(), "test program not built"
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert "quant_conv_test passed" in res.stdout


def algos_for(x, w, conv):
    n, h, wd, c = x.shape
    k, r, s, _ = w.shape
    out = ["auto", "direct"]
    for a in ("igemm", "stem", "band", "dot4"):
        d = M.make_desc(x.shape, w.shape, stride=conv[2:4], padding=conv[0:2], dilation=conv[4:6], groups=conv[6],
                        algo=a)
        try:
            M.plan(d)
            out.append(a)
        except M.MiqError:
            pass
    return out


def conv_kwargs(conv):
    return dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=conv[6])


def test_int8_accumulators_every_algo(device):
    ran = set()
    for name, c in cases.int8_cases().items():
        xd, wd = dev(c["x"], device), dev(c["w"], device)
        for algo in algos_for(c["x"], c["w"], c["conv"]):
            y = M.qconv2d_nhwc_i8_acc32(xd, wd, algo=algo, **conv_kwargs(c["conv"]))
            torch.cuda.synchronize()
            np.testing.assert_array_equal(y.cpu().numpy(), c["y"], err_msg=f"{name} {algo}")
            ran.add(algo)
    assert ran == {"auto", "direct", "igemm", "stem", "band", "dot4"}


def requant_inputs(k, seed):
    bias = W.fill_i32_uniform(k, seed, -1024, 1024)
    ws = W.fill_f32_uniform(k, seed + 1, 1e-3, 1e-2)
    return bias, ws


def test_int8_requant_and_dequant_every_algo(device):
    for idx, (name, c) in enumerate(cases.int8_cases().items()):
        k = c["w"].shape[0]
        bias, ws = requant_inputs(k, 1000 + idx)
        in_scale = 0.02 if name != "extreme_values" else 2e-5
        xd, wd, bd, sd = dev(c["x"], device), dev(c["w"], device), dev(bias, device), dev(ws, device)
        for relu in (False, True):
            want_q = oracle.requant_i8(c["y"], bias, ws, in_scale, 1.0, relu)
            want_f = oracle.dequant_f32(c["y"], bias, ws, in_scale, 1.0, relu)
            for algo in algos_for(c["x"], c["w"], c["conv"]):
                q = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=relu, in_scale=in_scale, algo=algo, **conv_kwargs(c["conv"]))
                f = M.qconv2d_nhwc_i8_dequant(xd, wd, bd, sd, relu=relu, in_scale=in_scale, algo=algo,
                                              **conv_kwargs(c["conv"]))
                torch.cuda.synchronize()
                np.testing.assert_array_equal(q.cpu().numpy(), want_q, err_msg=f"{name} {algo} relu={relu}")
                got_f = f.cpu().numpy()
                np.testing.assert_array_equal(got_f.view(np.uint32), want_f.view(np.uint32),
                                              err_msg=f"{name} {algo} relu={relu} (fp32, tolerance 1 ulp; bits compared)")
        # no bias pointer: bias treated as 0
        q = M.qconv2d_nhwc_i8(xd, wd, None, sd, in_scale=in_scale, **conv_kwargs(c["conv"]))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(q.cpu().numpy(), oracle.requant_i8(c["y"], None, ws, in_scale, 1.0, False))


@pytest.fixture(scope="module")
def config_data():
    return {}


@pytest.mark.parametrize("name", list(W.WORKLOADS))
def test_config_full_size(device, name):
    wl = W.WORKLOADS[name]
    g = cases.config_goldens()[name]
    inp = wl.inputs()
    xd, wd = dev(inp["x"], device), dev(inp["w"], device)
    bd, sd = dev(inp["bias"], device), dev(inp["w_scale"], device)
    kw = dict(stride=wl.stride, padding=wl.pad)
    acc = M.qconv2d_nhwc_i8_acc32(xd, wd, **kw)
    torch.cuda.synchronize()
    acc_h = acc.cpu().numpy()
    assert list(acc_h.shape) == g["shape"]
    np.testing.assert_array_equal(acc_h.reshape(-1)[::g["sample_stride"]], g["samples"])
    assert hashlib.sha256(acc_h.tobytes()).hexdigest() == g["acc_sha256"], f"{name}: accumulators differ"
    # fused int8 output and fp32 view against the oracle's epilogue on the golden accumulators
    q = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=wl.relu, in_scale=wl.in_scale, out_scale=wl.out_scale, **kw)
    f = M.qconv2d_nhwc_i8_dequant(xd, wd, bd, sd, relu=wl.relu, in_scale=wl.in_scale, out_scale=wl.out_scale, **kw)
    torch.cuda.synchronize()
    want_q = oracle.requant_i8(acc_h, inp["bias"], inp["w_scale"], wl.in_scale, wl.out_scale, wl.relu)
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)
    want_f = oracle.dequant_f32(acc_h, inp["bias"], inp["w_scale"], wl.in_scale, wl.out_scale, wl.relu)
    np.testing.assert_array_equal(f.cpu().numpy().view(np.uint32), want_f.view(np.uint32))
    # the VALU kernels agree on the full problem too: the direct one and the v_dot4 one
    acc2 = M.qconv2d_nhwc_i8_acc32(xd, wd, algo="direct", **kw)
    torch.cuda.synchronize()
    assert hashlib.sha256(acc2.cpu().numpy().tobytes()).hexdigest() == g["acc_sha256"]
    acc3 = M.qconv2d_nhwc_i8_acc32(xd, wd, algo="dot4", **kw)
    q3 = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=wl.relu, in_scale=wl.in_scale, out_scale=wl.out_scale, algo="dot4",
                           **kw)
    torch.cuda.synchronize()
    assert hashlib.sha256(acc3.cpu().numpy().tobytes()).hexdigest() == g["acc_sha256"], f"{name}: dot4 accumulators"
    np.testing.assert_array_equal(q3.cpu().numpy(), want_q)


def test_stride_two_is_subsampled_stride_one_full_size(device):
    wl = W.WORKLOADS["down_s2"]
    inp = wl.inputs()
    xd, wd = dev(inp["x"], device), dev(inp["w"], device)
    s2 = M.qconv2d_nhwc_i8_acc32(xd, wd, stride=2, padding=1)
    s1 = M.qconv2d_nhwc_i8_acc32(xd, wd, stride=1, padding=1)
    torch.cuda.synchronize()
    assert torch.equal(s2, s1[:, ::2, ::2, :].contiguous())


def test_linearity_full_size(device):
    wl = W.WORKLOADS["r50_3x3"]
    inp = wl.inputs()
    x = torch.from_numpy(inp["x"]).to(device)
    a = (x // 2).to(torch.int8)
    b = (x - a).to(torch.int8)
    wd = dev(inp["w"], device)
    ya = M.qconv2d_nhwc_i8_acc32(a.contiguous(), wd, padding=1)
    yb = M.qconv2d_nhwc_i8_acc32(b.contiguous(), wd, padding=1)
    yx = M.qconv2d_nhwc_i8_acc32(x, wd, padding=1)
    torch.cuda.synchronize()
    assert torch.equal(ya + yb, yx)


def test_side_stream_and_repeat_launches(device):
    wl = W.WORKLOADS["tiny"]
    inp = wl.inputs()
    xd, wd = dev(inp["x"], device), dev(inp["w"], device)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        outs = [M.qconv2d_nhwc_i8_acc32(xd, wd, padding=1) for _ in range(5)]
    s.synchronize()
    for y in outs:
        np.testing.assert_array_equal(y.cpu().numpy(), cases.c1_acc())


def test_unaligned_tensors_fall_back_exactly(device):
    wl = W.WORKLOADS["tiny"]
    inp = wl.inputs()
    buf = torch.zeros(inp["x"].size + 1, dtype=torch.int8, device=device)
    xv = buf[1:].view(inp["x"].shape)
    xv.copy_(torch.from_numpy(inp["x"]).to(device))
    wd = dev(inp["w"], device)
    assert M.plan(M.make_desc(xv.shape, wd.shape, padding=1)) == "igemm"  # judged for aligned buffers
    y = M.qconv2d_nhwc_i8_acc32(xv, wd, padding=1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), cases.c1_acc())
    with pytest.raises(M.MiqError, match="aligned"):
        M.qconv2d_nhwc_i8_acc32(xv, wd, padding=1, algo="igemm")


@pytest.mark.parametrize("dil", [(-1, -1), (1, -1), (-1, 1)])
def test_nonpositive_dilation_auto_matches_oracle(device, dil):
    """Negative dilation walks the taps backwards; the reference's CPU definition and
    infer_conv_shape accept it, so AUTO (which resolves to the direct kernel) must agree."""
    x = W.fill_i8_uniform(1 * 8 * 8 * 64, 71, -128, 127).reshape(1, 8, 8, 64)
    w = W.fill_i8_uniform(128 * 3 * 3 * 64, 72, -127, 127).reshape(128, 3, 3, 64)
    conv = (1, 1, 1, 1, dil[0], dil[1], 1)
    want = oracle.conv_i8_acc(x, w, conv)
    y = M.qconv2d_nhwc_i8_acc32(dev(x, device), dev(w, device), **conv_kwargs(conv))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), want)


def test_empty_batch(device):
    x = torch.zeros((0, 8, 8, 32), dtype=torch.int8, device=device)
    w = torch.zeros((16, 3, 3, 32), dtype=torch.int8, device=device)
    y = M.qconv2d_nhwc_i8_acc32(x, w, padding=1)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, 8, 8, 16)


def test_non_finite_scales_follow_the_definition(device):
    # NaN -> lo, +inf -> 127 (acc > 0) / lo (acc < 0), 0 * inf -> NaN -> lo; every kernel family
    c = cases.int8_cases()["c16_k32_3x3"]
    k = c["w"].shape[0]
    ws = np.full(k, 5e-3, np.float32)
    ws[0], ws[1], ws[2], ws[3] = np.nan, np.inf, -np.inf, 0.0
    bias = np.zeros(k, np.int32)
    bias[4] = -c["y"][..., 4].max() - 1   # pushes every value of channel 4 below lo
    xd, wd, bd, sd = dev(c["x"], device), dev(c["w"], device), dev(bias, device), dev(ws, device)
    for relu in (False, True):
        want = oracle.requant_i8(c["y"], bias, ws, 0.02, 1.0, relu)
        for algo in algos_for(c["x"], c["w"], c["conv"]):
            q = M.qconv2d_nhwc_i8(xd, wd, bd, sd, relu=relu, in_scale=0.02, algo=algo, **conv_kwargs(c["conv"]))
            torch.cuda.synchronize()
            np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"{algo} relu={relu}")
