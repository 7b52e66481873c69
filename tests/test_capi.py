"""The C-ABI library without a GPU: it loads, exports every declared symbol (C and the
C++ drop-in ABI), and validates arguments on the host exactly like the reference."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
import my_own_cnn_amd as M
from my_own_cnn_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", str(M.LIB_PATH)], check=True, capture_output=True,
                         text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.strip()}


def declared_c_functions():
    text = (ROOT / "include" / "miq_qconv.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(miq_[a-z0-9_]+)\s*\(", text))


def test_every_declared_c_symbol_is_exported_and_bound():
    decl = declared_c_functions()
    assert len(decl) >= 13
    assert decl <= exported()
    assert decl == set(_capi.SIGNATURES)
    lib = M.lib()
    for name in decl:
        assert getattr(lib, name) is not None
    assert lib.miq_version() == 100


def test_cpp_dropin_abi_is_exported():
    # mangled names a caller compiled against the reference's own conv_types.h needs
    need = set((GOLDEN / "dropin_symbols.txt").read_text().split())
    assert len(need) == 6
    assert need <= exported()


def test_cpp_additions_are_exported():
    demangled = subprocess.run(["c++filt"], input="\n".join(sorted(exported())), capture_output=True,
                               text=True).stdout
    for fn in ["launch_fprop_nhwc_qi8(", "launch_fprop_nhwc_qi8_acc32(", "launch_fprop_nhwc_qi8_dequant(",
               "HipEventTimer::start()", "HipEventTimer::stop_ms()"]:
        assert fn in demangled, fn


def test_no_cpu_convolution_in_the_product():
    syms = exported()
    assert not any("cpu_fprop" in s or "orc_" in s for s in syms)


def test_status_strings():
    lib = M.lib()
    assert lib.miq_status_string(0) == b"success"
    assert lib.miq_status_string(3) == b"unsupported by the requested algorithm"
    assert lib.miq_status_string(99) == b"unknown status"


SHAPES = [
    # n, h, w, c, r, s, k, conv7
    (1, 5, 5, 4, 3, 3, 4, (1, 1, 1, 1, 1, 1, 0)),
    (1, 5, 5, 4, 3, 3, 4, (1, 1, 1, 1, 1, 1, 3)),
    (1, 5, 5, 6, 3, 3, 4, (1, 1, 1, 1, 1, 1, 3)),
    (1, 2, 2, 4, 5, 5, 4, (0, 0, 1, 1, 1, 1, 1)),
    (1, 5, 5, 4, 3, 3, 4, (1, 1, 0, 1, 1, 1, 1)),
    (1, 5, 5, 4, 3, 3, 4, (1, 1, 1, -2, 1, 1, 1)),
    (2, 9, 7, 8, 3, 2, 6, (1, 0, 2, 1, 2, 1, 2)),
    (1, 1, 1, 1, 1, 1, 1, (0, 0, 1, 1, 1, 1, 1)),
    (1, 3, 3, 2, 7, 7, 2, (3, 3, 2, 2, 1, 1, 1)),
    (1, 0, 4, 2, 1, 1, 2, (1, 0, 1, 1, 1, 1, 1)),
    (1, 4, 4, 2, 3, 3, 2, (-1, 0, 1, 1, 1, 1, 1)),
]


def reference_shape(n, h, w, c, r, s, k, conv):
    lib = oracle.ref()
    lib.ref_infer_conv_shape.argtypes = [C.c_int] * 7 + [C.c_void_p, C.c_void_p, C.c_void_p]
    cv = np.array(conv, np.int32)
    ho, wo = C.c_int(), C.c_int()
    if lib.ref_infer_conv_shape(n, h, w, c, r, s, k, cv.ctypes.data, C.byref(ho), C.byref(wo)) != 0:
        return lib.ref_last_error().decode()
    return (ho.value, wo.value)


def ours_shape(n, h, w, c, r, s, k, conv):
    try:
        return M.infer_conv_shape(n, h, w, c, r, s, k, M.Conv2DParams(*conv))
    except M.MiqError as e:
        assert e.status == _capi.MIQ_ERR_INVALID_ARGUMENT
        return str(e).split(": ", 1)[1].rsplit(" (status", 1)[0]


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref (the reference's own headers) not built here")
@pytest.mark.parametrize("shape", SHAPES)
def test_shape_validation_matches_reference(shape):
    assert ours_shape(*shape) == reference_shape(*shape)


def test_shape_validation_messages():
    assert ours_shape(*SHAPES[0]) == "groups must be > 0"
    assert ours_shape(*SHAPES[1]) == "input channels must be divisible by groups"
    assert ours_shape(*SHAPES[2]) == "output channels must be divisible by groups"
    assert ours_shape(*SHAPES[3]) == "invalid output size (negative numerator)"
    assert ours_shape(*SHAPES[4]) == "stride must be > 0"
    assert ours_shape(*SHAPES[6]) == (4, 6)  # (9 + 2 - 2*2 - 1) // 2 + 1, (7 - 1 - 1) + 1


def test_block_shape_validation():
    bp = M.BlockConv2DParams(M.Conv2DParams(1, 1, 1, 1, 1, 1, 1), 2, 3)
    assert M.infer_block_conv_shape(2, 6, 6, 4, 3, 3, 5, bp) == (6, 6, 3, 2)
    with pytest.raises(M.MiqError, match="Ho/Wo divisible by block grid"):
        M.infer_block_conv_shape(2, 6, 6, 4, 3, 3, 5, M.BlockConv2DParams(M.Conv2DParams(), 4, 3))
    with pytest.raises(M.MiqError, match="block_by and block_bx must be > 0"):
        M.infer_block_conv_shape(2, 6, 6, 4, 3, 3, 5, M.BlockConv2DParams(M.Conv2DParams(), 0, 3))


def test_entry_points_reject_before_touching_the_gpu():
    lib = M.lib()
    p = M.Conv2DParams()
    fake = 0x1000  # never dereferenced: validation fails first
    st = lib.miq_fprop_nhwc_qi32_u8(fake, fake, fake, 1, 5, 5, 4, 3, 3, 4, C.byref(M.Conv2DParams(groups=0)),
                                    fake, fake, None)
    assert st == _capi.MIQ_ERR_INVALID_ARGUMENT
    assert lib.miq_last_error_message() == b"groups must be > 0"
    st = lib.miq_fprop_nhwc_qi32_s5(fake, fake, fake, 1, 5, 5, 4, 3, 3, 4, C.byref(p), None, fake, None)
    assert st == _capi.MIQ_ERR_NULL_POINTER
    st = lib.miq_fprop_nhwc_qi32_s5(fake, fake, None, 1, 5, 5, 4, 3, 3, 4, C.byref(p), fake, fake, None)
    assert st == _capi.MIQ_ERR_NULL_POINTER
    assert lib.miq_qconv2d_nhwc_i8(None, fake, fake, None, fake, fake, None) == _capi.MIQ_ERR_NULL_POINTER
    d = M.make_desc((1, 8, 8, 3), (4, 3, 3, 3), padding=1, algo="igemm")
    assert lib.miq_qconv2d_nhwc_i8(C.byref(d), fake, fake, None, fake, fake, None) == _capi.MIQ_ERR_UNSUPPORTED
    assert b"% 16" in lib.miq_last_error_message()
    d = M.make_desc((1, 8, 8, 32), (4, 3, 3, 32), padding=1, algo="stem")
    assert lib.miq_qconv2d_nhwc_i8(C.byref(d), fake, fake, None, fake, fake, None) == _capi.MIQ_ERR_UNSUPPORTED
    d = M.make_desc((1, 8, 8, 32), (4, 3, 3, 32), padding=1)
    assert lib.miq_qconv2d_nhwc_i8(C.byref(d), fake, fake, None, None, fake, None) == _capi.MIQ_ERR_NULL_POINTER
    d = M.make_desc((1, 8, 8, 32), (4, 3, 3, 32), padding=1, out_scale=0.0)
    assert lib.miq_qconv2d_nhwc_i8(C.byref(d), fake, fake, None, fake, fake, None) == _capi.MIQ_ERR_INVALID_ARGUMENT
    d = M.make_desc((1, 8, 8, 32), (4, 3, 3, 32), padding=1, algo=99)
    assert lib.miq_qconv2d_nhwc_i8_acc32(C.byref(d), fake, fake, fake, None) == _capi.MIQ_ERR_INVALID_ARGUMENT
    # the pipe kernel writes int8 outputs only
    d = M.make_desc((1, 8, 8, 64), (64, 3, 3, 64), padding=1, algo="pipe")
    assert lib.miq_qconv2d_nhwc_i8_acc32(C.byref(d), fake, fake, fake, None) == _capi.MIQ_ERR_UNSUPPORTED
    assert b"int8 outputs only" in lib.miq_last_error_message()
    d = M.make_desc((-1, 8, 8, 32), (4, 3, 3, 32), padding=1)
    assert lib.miq_qconv2d_nhwc_i8_acc32(C.byref(d), fake, fake, fake, None) == _capi.MIQ_ERR_INVALID_ARGUMENT


def test_empty_batch_is_a_no_op():
    # n == 0: valid, nothing to compute, nothing enqueued (no GPU needed)
    lib = M.lib()
    d = M.make_desc((0, 8, 8, 32), (4, 3, 3, 32), padding=1)
    assert lib.miq_qconv2d_nhwc_i8_acc32(C.byref(d), None, None, None, None) == _capi.MIQ_ERR_NULL_POINTER
    fake = 0x1000
    assert lib.miq_qconv2d_nhwc_i8_acc32(C.byref(d), None, fake, None, None) == _capi.MIQ_OK


def test_python_mirror_errors():
    with pytest.raises(RuntimeError, match="requires non-null quantization parameters"):
        M.launch_fprop_nhwc_qi32(M.DataType.LinQuantU8, 1, 1, 1, 1, 5, 5, 4, 3, 3, 4, None, None, 1)
    with pytest.raises(TypeError, match="supports only LinQuantU8 and LinQuantS5"):
        M.launch_fprop_nhwc_qi32(M.DataType.LinQuantI8, 1, 1, 1, 1, 5, 5, 4, 3, 3, 4, None, 1, 1)


@pytest.mark.parametrize("name,algo", [("tiny", "igemm"), ("r50_3x3", "band"), ("r50_1x1", "pointwise"),
                                       ("down_s2", "stream"), ("stem", "stem_s2d")])
def test_plan_of_the_workloads(name, algo):
    wl = M.WORKLOADS[name]
    d = M.make_desc((wl.n, wl.h, wl.w, wl.c), (wl.k, wl.r, wl.s, wl.c), stride=wl.stride, padding=wl.pad,
                    relu=wl.relu, in_scale=wl.in_scale)
    assert M.plan(d) == algo


def test_qi32_workspace_size():
    """The caller-workspace size of the float-code path (no GPU access): the row-band kernel's
    filter prepass output on C2 (9 K-blocks of one 64-channel tile: 4 KB of int8 fragments and
    a 4-byte range flag each), the stream route's on C4 (the zero-padded int8 copy of the input,
    32 x 58 x 58 x 128 bytes, then the int8 filter 256 x 1152, per-channel sums 256 x 4, per-image
    parameters 32 x 16 and 3396 flags, each part 256-byte aligned), and none for the kernels
    that need none."""
    c2 = M.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    c4 = M.Conv2DParams(1, 1, 2, 2, 1, 1, 1)
    assert M.qi32_workspace_size(32, 56, 56, 64, 3, 3, 64, c2) == 9 * 4096 + 9 * 4
    assert M.qi32_workspace_size(32, 56, 56, 64, 3, 3, 64, c2, algo="band") == 9 * 4096 + 9 * 4
    padded = 32 * 58 * 58 * 128
    assert padded % 256 == 0
    route = padded + 256 * 1152 + 256 * 4 + 32 * 16 + 3396 * 4
    assert M.qi32_workspace_size(32, 56, 56, 128, 3, 3, 256, c4) == (route + 255) // 256 * 256
    for algo in ("igemm", "direct"):
        assert M.qi32_workspace_size(32, 56, 56, 64, 3, 3, 64, c2, algo=algo) == 0
    assert M.qi32_workspace_size(1, 32, 32, 16, 3, 3, 32, c2) == 0  # C1 runs the implicit GEMM
    with pytest.raises(M.MiqError, match="band"):
        M.qi32_workspace_size(1, 32, 32, 16, 3, 3, 32, c2, algo="band")  # c % 64 != 0
    lib = M.lib()
    out = C.c_size_t(5)
    assert lib.miq_fprop_nhwc_qi32_workspace_size(32, 56, 56, 64, 3, 3, 64, C.byref(c2), 99, C.byref(out)) == 2
    assert lib.miq_fprop_nhwc_qi32_workspace_size(32, 56, 56, 64, 3, 3, 64, C.byref(c2), 0, None) == 1


def test_qi32_ws_validates_before_launch():
    """The caller-workspace entry point checks its workspace on the host before anything is
    enqueued: too small or NULL where one is needed is an error (no GPU access needed)."""
    lib = M.lib()
    c2 = M.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    need = M.qi32_workspace_size(32, 56, 56, 64, 3, 3, 64, c2)
    fake = C.c_void_p(1 << 20)  # never dereferenced: validation fails first
    st = lib.miq_fprop_nhwc_qi32_ws(0, fake, fake, fake, 32, 56, 56, 64, 3, 3, 64, C.byref(c2), fake, fake, 4,
                                    fake, need - 1, None)
    assert st == 2 and b"smaller than miq_fprop_nhwc_qi32_workspace_size" in lib.miq_last_error_message()
    st = lib.miq_fprop_nhwc_qi32_ws(0, fake, fake, fake, 32, 56, 56, 64, 3, 3, 64, C.byref(c2), fake, fake, 4,
                                    None, need, None)
    assert st == 1 and b"workspace pointer is NULL" in lib.miq_last_error_message()
    st = lib.miq_fprop_nhwc_qi32_ws(2, fake, fake, fake, 32, 56, 56, 64, 3, 3, 64, C.byref(c2), fake, fake, 0,
                                    fake, need, None)
    assert st == 2 and b"qp_kind" in lib.miq_last_error_message()


@pytest.mark.parametrize("dil", [(-1, -1), (1, -1), (-1, 1), (0, 1), (1, 0)])
def test_plan_never_sends_nonpositive_dilation_to_mfma_kernels(dil):
    """infer_conv_shape accepts dilation <= 0 (as the reference's does); only the direct
    kernel walks such taps, so AUTO must resolve there and the MFMA kernels must refuse."""
    x_shape, w_shape = (1, 8, 8, 64), (128, 3, 3, 64)
    try:
        d = M.make_desc(x_shape, w_shape, padding=1, dilation=dil)
        auto = M.plan(d)
    except M.MiqError:
        return  # the shape itself is rejected: nothing runs
    assert auto == "direct", (dil, auto)
    for algo in ("band", "stream", "igemm", "stem", "pipe"):
        with pytest.raises(M.MiqError):
            M.plan(M.make_desc(x_shape, w_shape, padding=1, dilation=dil, algo=algo))


def test_qparams_byte_layout():
    a = M.qparams_array(M.DataType.LinQuantU8, [37, 66], [0.25, 0.35])
    raw = a.tobytes()
    assert len(raw) == 24 and raw[0] == 37 and raw[12] == 66
    assert np.frombuffer(raw[4:8], np.float32)[0] == np.float32(0.25)
    b = M.qparams_array(M.DataType.LinQuantS5, [-5, 2], n_bins=31)
    raw = b.tobytes()
    assert len(raw) == 16 and raw[0] == 0xFB and raw[1] == 31 and raw[8] == 2


HARNESS_CASES = {
    "exact_equal": ([1, -2, 3.5], [1, -2, 3.5], 0, 0),
    "one_off": ([100, 200, 300], [100, 201, 300], 0, 0),
    "within_abs": ([1, 2], [1.00005, 2], 1e-4, 0),
    "within_rel": ([1000, 2], [1000.5, 2], 1e-4, 1e-3),
    "zero_ref": ([0, 0], [1e-7, 3e-3], 1e-4, 1e-3),
    "tiny_ref": ([1e-7, 5], [2e-7, 5], 0, 0),
    "negative": ([-4, -8], [-4.004, -8], 1e-4, 1e-3),
    "empty": ([], [], 0, 0),
}


def test_cpp_harness_verify_tensors():
    exe = ROOT / "tests" / "cpp" / "bin" / "harness_test"
    assert exe.exists(), "build with __graft_entry__.build()"
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()
    got = {ln.split()[0]: ln.split()[1:] for ln in lines if ln.split()[0] in HARNESS_CASES}
    assert set(got) == set(HARNESS_CASES)
    expect_pass = {"exact_equal": 1, "one_off": 0, "within_abs": 1, "within_rel": 1, "zero_ref": 0, "tiny_ref": 0,
                   "negative": 0, "empty": 1}
    for name, (a, b, ae, re_) in HARNESS_CASES.items():
        g = got[name]
        assert int(g[4]) == expect_pass[name], name
        if oracle.ref() is not None:  # the reference's own verify_tensors on the same vectors
            r = oracle.ref_verify_tensors(np.array(a, np.float32), np.array(b, np.float32), ae, re_)
            assert int(r["passed"]) == int(g[4]), name
            assert np.float32(r["max_abs_err"]) == np.float32(float(g[0])), name
            assert np.float32(r["max_rel_err"]) == np.float32(float(g[1])), name
            assert (r["max_abs_idx"], r["max_rel_idx"]) == (int(g[2]), int(g[3])), name
    assert "size_mismatch_throws 1" in lines
    assert [ln for ln in lines if ln.startswith("shape")] == [
        "shape error: groups must be > 0", "shape error: input channels must be divisible by groups",
        "shape error: output channels must be divisible by groups",
        "shape error: invalid output size (negative numerator)", "shape error: stride must be > 0"]


def test_bmm_dropin_symbol_is_exported():
    # bmm.h declares it inside extern "C": the unmangled name is the drop-in ABI
    assert "bmm_matmul_i32" in exported()


def test_bmm_rejects_before_touching_the_gpu():
    lib = M.lib()
    p = C.c_void_p(256)  # never dereferenced: every call below fails validation or has no work
    for args, status in [((p, p, p, -1, 2, 2, 2, 0, 0), _capi.MIQ_ERR_INVALID_ARGUMENT),
                         ((p, p, p, 1, 2, -2, 2, 0, 0), _capi.MIQ_ERR_INVALID_ARGUMENT),
                         ((p, p, p, 1, 2, 2, -1, 1, 1), _capi.MIQ_ERR_INVALID_ARGUMENT),
                         ((p, p, None, 1, 2, 2, 2, 0, 0), _capi.MIQ_ERR_NULL_POINTER),
                         ((None, p, p, 1, 2, 2, 2, 0, 0), _capi.MIQ_ERR_NULL_POINTER),
                         ((p, None, p, 1, 2, 2, 2, 0, 1), _capi.MIQ_ERR_NULL_POINTER),
                         ((p, p, p, 1, 2 ** 31 - 1, 2, 2, 0, 0), _capi.MIQ_ERR_UNSUPPORTED),
                         ((p, p, p, 1, 2 ** 24, 2 ** 16, 2, 0, 0), _capi.MIQ_ERR_UNSUPPORTED),
                         ((None, None, None, 0, 5, 5, 5, 0, 0), _capi.MIQ_OK),
                         ((None, None, None, 3, 0, 5, 5, 0, 0), _capi.MIQ_OK),
                         ((None, None, None, 3, 5, 0, 5, 1, 0), _capi.MIQ_OK)]:
        assert lib.miq_bmm_i32(*args, None) == status, args
    assert lib.miq_bmm_i32(p, p, p, 1, 2, 2, -1, 0, 0, None) == _capi.MIQ_ERR_INVALID_ARGUMENT
    assert b"extents" in lib.miq_last_error_message()
    # the void drop-in records the reason and enqueues nothing
    drop = lib.bmm_matmul_i32
    drop.restype = None
    drop.argtypes = [C.c_void_p] * 3 + [C.c_int] * 6
    drop(p, p, None, 1, 2, 2, 2, 0, 0)
    assert b"output pointer C is NULL" in lib.miq_last_error_message()


def test_bmm_python_mirror_errors():
    with pytest.raises(M.MiqError, match="extents must be >= 0"):
        M.bmm_matmul_i32(256, 256, 256, 1, -3, 2, 2, 0, 0, stream=0)
    M.bmm_matmul_i32(None, None, None, 0, 4, 4, 4, 0, 0, stream=0)  # empty batch: no work, no error


def test_fp32_conv_dropin_and_validation():
    need = "_Z17launch_fprop_nhwcPKfS0_PfiiiiiiiRK12Conv2DParams"  # the reference's conv_types.h:287-289
    assert need in exported()
    lib = M.lib()
    p = C.c_void_p(256)  # never dereferenced: each call fails validation or has no work
    ok = _capi.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    bad = _capi.Conv2DParams(1, 1, 0, 1, 1, 1, 1)
    assert lib.miq_fprop_nhwc_f32(p, p, p, 1, 5, 5, 4, 3, 3, 4, C.byref(bad), 0, None) == _capi.MIQ_ERR_INVALID_ARGUMENT
    assert b"stride must be > 0" in lib.miq_last_error_message()
    assert lib.miq_fprop_nhwc_f32(p, p, None, 1, 5, 5, 4, 3, 3, 4, C.byref(ok), 0, None) == _capi.MIQ_ERR_NULL_POINTER
    assert lib.miq_fprop_nhwc_f32(p, p, p, 1, 5, 5, 4, 3, 3, 4, C.byref(ok), 7, None) == _capi.MIQ_ERR_INVALID_ARGUMENT
    assert lib.miq_fprop_nhwc_f32(p, p, p, 1, 5, 5, 6, 3, 3, 4, C.byref(ok), 2, None) == _capi.MIQ_ERR_UNSUPPORTED
    assert b"% 4" in lib.miq_last_error_message()
    assert lib.miq_fprop_nhwc_f32(None, p, None, 0, 5, 5, 4, 3, 3, 4, C.byref(ok), 0, None) == _capi.MIQ_OK  # n == 0
    with pytest.raises(M.MiqError, match="stride must be > 0"):
        M.launch_fprop_nhwc(256, 256, 256, 1, 5, 5, 4, 3, 3, 4, (1, 1, 0, 1, 1, 1, 1), stream=0)


def test_fp32_grad_workspace_query_and_validation():
    lib = M.lib()
    ok = _capi.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    out = C.c_size_t(123)
    # the ordered MFMA grad of the conv_bench 56x56 shape splits its 100352 pixels: a workspace
    assert lib.miq_grad_nhwc_f32_workspace_size(32, 56, 56, 64, 3, 3, 64, C.byref(ok), 0, C.byref(out)) == 0
    assert out.value > 0 and out.value % (64 * 576 * 4) == 0
    for algo in ("atomic", "direct"):  # no partial tiles kept
        assert M.grad_workspace_size(32, 56, 56, 64, 3, 3, 64, (1, 1, 1, 1, 1, 1, 1), algo) == 0
    assert M.grad_workspace_size(1, 4, 4, 4, 1, 1, 4, (0, 0, 1, 1, 1, 1, 1)) == 0  # one split writes dw
    assert lib.miq_grad_nhwc_f32_workspace_size(1, 5, 5, 4, 3, 3, 4, C.byref(ok), 0, None) == _capi.MIQ_ERR_NULL_POINTER
    assert lib.miq_grad_nhwc_f32_workspace_size(1, 5, 5, 4, 3, 3, 4, C.byref(ok), 9, C.byref(out)) == \
        _capi.MIQ_ERR_INVALID_ARGUMENT
    assert b"ATOMIC" in lib.miq_last_error_message()
    # the caller-workspace form validates before touching the GPU
    p = C.c_void_p(256)
    need = M.grad_workspace_size(32, 56, 56, 64, 3, 3, 64, (1, 1, 1, 1, 1, 1, 1))
    assert lib.miq_grad_nhwc_f32_ws(p, p, p, 32, 56, 56, 64, 3, 3, 64, C.byref(ok), 0, None, need, None) == \
        _capi.MIQ_ERR_NULL_POINTER
    assert lib.miq_grad_nhwc_f32_ws(p, p, p, 32, 56, 56, 64, 3, 3, 64, C.byref(ok), 0, p, need - 4, None) == \
        _capi.MIQ_ERR_INVALID_ARGUMENT
    assert b"smaller" in lib.miq_last_error_message()
    assert lib.miq_grad_nhwc_f32_ws(p, p, None, 1, 5, 5, 4, 3, 3, 0, C.byref(ok), 0, None, 0, None) == _capi.MIQ_OK  # k == 0


def test_plan_f32_names_the_kernel_each_pass_runs():
    # the fp32 passes' dispatch, answered by the library without touching the GPU
    r50 = (32, 56, 56, 64, 3, 3, 64)
    dw = _capi.Conv2DParams(1, 1, 1, 1, 1, 1, 64)  # depthwise: groups = C = K
    assert M.plan_f32("fprop", *r50) == "igemm"
    assert M.plan_f32("fprop", 8, 28, 28, 64, 3, 3, 32) == "igemm32"  # K per group <= 32
    assert M.plan_f32("fprop", *r50, dw) == "depthwise"
    assert M.plan_f32("fprop", *r50, algo="direct") == "direct"
    assert M.plan_f32("bprop", *r50) == "bprop_igemm"
    assert M.plan_f32("bprop", *r50, dw) == "depthwise"
    assert M.plan_f32("bprop", *r50, dw, algo="direct") == "direct"
    assert M.plan_f32("bprop", 8, 28, 28, 32, 3, 3, 32, _capi.Conv2DParams(1, 1, 2, 2, 1, 1, 1)) == "direct"
    assert M.plan_f32("grad", *r50) == "grad_igemm"
    assert M.plan_f32("grad", *r50, dw) == "grad_depthwise"
    assert M.plan_f32("grad", *r50, algo="direct") == "direct"
    lib = M.lib()
    ok = _capi.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    out = C.c_int32(-1)
    assert lib.miq_plan_f32(3, *r50, C.byref(ok), 0, C.byref(out)) == _capi.MIQ_ERR_INVALID_ARGUMENT
    assert lib.miq_plan_f32(0, *r50, C.byref(ok), _capi.MIQ_ALGO_STREAM, C.byref(out)) == _capi.MIQ_ERR_INVALID_ARGUMENT
    assert lib.miq_plan_f32(0, *r50, C.byref(ok), 0, None) == _capi.MIQ_ERR_NULL_POINTER
    bad = _capi.Conv2DParams(1, 1, 0, 1, 1, 1, 1)  # stride 0: the shape check rejects it
    assert lib.miq_plan_f32(0, *r50, C.byref(bad), 0, C.byref(out)) != _capi.MIQ_OK
    with pytest.raises(ValueError, match="algo"):
        M.plan_f32("fprop", *r50, algo="stream")
    with pytest.raises(ValueError, match="op"):
        M.plan_f32("wgrad", *r50)
    with pytest.raises(M.MiqError):
        M.plan_f32("fprop", 1, 2, 2, 16, 3, 3, 16, _capi.Conv2DParams(0, 0, 1, 1, 1, 1, 1))  # no output pixels


def test_blocked_fp32_dropins_and_validation():
    # the reference's launch_block_{fprop,bprop,grad}_nhwc (conv_types.h:296-304), same mangled names
    syms = exported()
    for need in ("_Z23launch_block_fprop_nhwcPKfS0_PfiiiiiiiRK17BlockConv2DParamsS0_13BlockBiasMode",
                 "_Z23launch_block_bprop_nhwcPKfS0_PfiiiiiiiRK17BlockConv2DParams",
                 "_Z22launch_block_grad_nhwcPKfS0_PfiiiiiiiRK17BlockConv2DParamsS1_13BlockBiasMode"):
        assert need in syms, need
    lib = M.lib()
    p = C.c_void_p(256)  # never dereferenced: each call fails validation or has no work
    conv = _capi.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    ok = _capi.BlockConv2DParams(conv, 2, 2)
    for fn, extra in ((lib.miq_block_fprop_nhwc_f32, (p, 0, 0)), (lib.miq_block_bprop_nhwc_f32, (0,)),
                      (lib.miq_block_grad_nhwc_f32, (p, 0, 0))):
        # an 8 x 8 output (3x3, pad 1) does not split into a 3 x 2 grid; a 0 grid is rejected outright
        for by, bx, msg in ((3, 2, b"divisible by block grid"), (0, 2, b"must be > 0")):
            bad = _capi.BlockConv2DParams(conv, by, bx)
            assert fn(p, p, p, 1, 8, 8, 4, 3, 3, 4, C.byref(bad), *extra, None) == _capi.MIQ_ERR_INVALID_ARGUMENT
            assert msg in lib.miq_last_error_message()
        assert fn(p, p, None, 1, 8, 8, 4, 3, 3, 4, C.byref(ok), *extra, None) == _capi.MIQ_ERR_NULL_POINTER
        assert fn(p, p, p, 1, 8, 8, 4, 3, 3, 4, None, *extra, None) == _capi.MIQ_ERR_NULL_POINTER
    # bias_mode and algo are checked before any launch
    assert lib.miq_block_fprop_nhwc_f32(p, p, p, 1, 8, 8, 4, 3, 3, 4, C.byref(ok), p, 2, 0, None) == \
        _capi.MIQ_ERR_INVALID_ARGUMENT
    assert b"bias_mode" in lib.miq_last_error_message()
    assert lib.miq_block_grad_nhwc_f32(p, p, p, 1, 8, 8, 4, 3, 3, 4, C.byref(ok), p, -1, 0, None) == \
        _capi.MIQ_ERR_INVALID_ARGUMENT
    assert lib.miq_block_bprop_nhwc_f32(p, p, p, 1, 8, 8, 4, 3, 3, 4, C.byref(ok), 9, None) == \
        _capi.MIQ_ERR_INVALID_ARGUMENT
    # c/groups == 2: no MFMA form
    assert lib.miq_block_fprop_nhwc_f32(p, p, p, 1, 8, 8, 2, 3, 3, 4, C.byref(ok), None, 0, 2, None) == \
        _capi.MIQ_ERR_UNSUPPORTED
    # empty batch: nothing to do for fprop / bprop
    assert lib.miq_block_fprop_nhwc_f32(None, p, None, 0, 8, 8, 4, 3, 3, 4, C.byref(ok), None, 0, 0, None) == _capi.MIQ_OK
    assert lib.miq_block_bprop_nhwc_f32(None, p, None, 0, 8, 8, 4, 3, 3, 4, C.byref(ok), 0, None) == _capi.MIQ_OK
    with pytest.raises(ValueError, match="bias_mode"):
        M.launch_block_fprop_nhwc(256, 256, 256, 1, 8, 8, 4, 3, 3, 4, ok, 256, "both", stream=0)


def test_plan_block_f32():
    conv = _capi.Conv2DParams(1, 1, 1, 1, 1, 1, 1)
    b22 = M.BlockConv2DParams(conv, 2, 2)
    assert M.plan_block_f32("fprop", 32, 56, 56, 64, 3, 3, 64, b22) == "igemm"
    assert M.plan_block_f32("bprop", 32, 56, 56, 64, 3, 3, 64, b22) == "bprop_igemm"
    assert M.plan_block_f32("grad", 32, 56, 56, 64, 3, 3, 64, b22) == "grad_igemm"
    # depthwise blocked: no depthwise kernel for blocked filters, the direct ones run
    dwp = M.BlockConv2DParams(_capi.Conv2DParams(1, 1, 1, 1, 1, 1, 64), 2, 2)
    assert M.plan_block_f32("fprop", 32, 56, 56, 64, 3, 3, 64, dwp) == "direct"
    assert M.plan_block_f32("grad", 32, 56, 56, 64, 3, 3, 64, dwp) == "grad_igemm"
    s2 = M.BlockConv2DParams(_capi.Conv2DParams(1, 1, 2, 2, 1, 1, 1), 2, 2)
    assert M.plan_block_f32("bprop", 32, 56, 56, 64, 3, 3, 64, s2) == "direct"
    with pytest.raises(M.MiqError, match="divisible"):
        M.plan_block_f32("fprop", 32, 56, 56, 64, 3, 3, 64, M.BlockConv2DParams(conv, 3, 2))


@pytest.mark.parametrize("shape,want", [
    (((32, 56, 56, 64), (8, 1, 1, 64), {}), "dot4"),           # 1x1, 8 output channels
    (((32, 28, 28, 512), (4, 1, 1, 512), {}), "dot4"),
    (((1, 56, 56, 64), (1, 1, 1, 64), {}), "dot4"),
    (((32, 112, 112, 16), (8, 3, 3, 16), {"padding": 1}), "dot4"),  # 3x3 with r*s*c/g = 144
    (((32, 56, 56, 64), (8, 3, 3, 64), {"padding": 1}), "igemm"),   # 576: the implicit GEMM measured faster
    (((32, 56, 56, 64), (12, 1, 1, 64), {}), "igemm"),         # 12 channels: equal, not taken
    (((32, 56, 56, 64), (16, 1, 1, 64), {}), "band"),          # band kernels win from 16 channels
    (((32, 224, 224, 3), (64, 7, 7, 3), {"padding": 3, "stride": 2}), "stem_s2d"),  # C = 3 stem stays on MFMA
])
def test_auto_takes_the_dot4_kernel_where_it_measured_faster(shape, want):
    xs, ws, kw = shape
    assert M.plan(M.make_desc(xs, ws, **kw)) == want


@pytest.mark.parametrize("xs,ws,kw,ok", [
    ((64, 28, 28, 128), (512, 1, 1, 128), {}, True),
    ((2, 7, 7, 64), (192, 1, 1, 64), {}, True),
    ((2, 7, 7, 64), (64, 3, 3, 64), {"padding": 1}, False),        # not 1x1
    ((2, 8, 8, 64), (64, 1, 1, 64), {"stride": 2}, False),         # strided
    ((2, 8, 8, 64), (64, 1, 1, 64), {"padding": 1}, False),        # padded
    ((2, 8, 8, 256), (64, 1, 1, 256), {}, False),                  # c = 256
    ((2, 8, 8, 64), (48, 1, 1, 64), {}, False),                    # k % 64 != 0
    ((2, 8, 8, 128), (128, 1, 1, 64), {"groups": 2}, False),       # grouped
])
def test_pointwise_planner(xs, ws, kw, ok):
    d = M.make_desc(xs, ws, algo="pointwise", **kw)
    if ok:
        assert M.plan(d) == "pointwise"
    else:
        with pytest.raises(M.MiqError):
            M.plan(d)


@pytest.mark.parametrize("xs,ws,kw,ok", [
    ((32, 224, 224, 3), (64, 7, 7, 3), {"stride": 2, "padding": 3}, True),
    ((2, 20, 16, 1), (128, 3, 3, 1), {"stride": 2, "padding": 1}, True),
    ((2, 20, 16, 3), (64, 7, 7, 3), {"stride": 1, "padding": 3}, False),   # stride 1
    ((2, 20, 16, 8), (64, 3, 3, 8), {"stride": 2, "padding": 1}, False),   # c > 4
    ((2, 20, 20, 3), (64, 7, 7, 3), {"stride": 2, "padding": 3}, False),   # w * c % 16 != 0
    ((2, 20, 16, 3), (48, 7, 7, 3), {"stride": 2, "padding": 3}, False),   # k % 64 != 0
    ((2, 40, 32, 1), (64, 9, 9, 1), {"stride": 2, "padding": 4}, False),   # 5 x 5 s2d taps > 16
    ((2, 20, 16, 3), (64, 3, 3, 3), {"stride": 2, "padding": 1, "dilation": 2}, False),
])
def test_stem_s2d_planner(xs, ws, kw, ok):
    d = M.make_desc(xs, ws, algo="stem_s2d", **kw)
    if ok:
        assert M.plan(d) == "stem_s2d"
    else:
        with pytest.raises(M.MiqError):
            M.plan(d)
