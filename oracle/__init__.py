"""CPU oracle of the quantized NHWC convolution - TEST INFRASTRUCTURE ONLY.

Loads oracle/liborc.so (the C restatement in qconv_oracle.c) and, when it was built,
oracle/_ref/libref_cpu.so (the reference's own cpu_ref.cpp, see oracle/Makefile).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package;
the product never does.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Optional, Sequence, Tuple

import numpy as np

HERE = Path(__file__).resolve().parent
ORC_PATH = HERE / "liborc.so"
REF_PATH = HERE / "_ref" / "libref_cpu.so"

_orc = None
_ref = None

_P = C.c_void_p
_I = C.c_int32


def build(reference_root: str = "/root/reference") -> None:
    """make -C oracle (the reference build only happens where its sources exist)."""
    subprocess.run(["make", "-C", str(HERE), "--no-print-directory", f"REF={reference_root}"], check=True,
                   stdout=subprocess.PIPE, stderr=subprocess.STDOUT)


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORC_PATH.exists():
            build()
        h = C.CDLL(str(ORC_PATH))
        h.orc_splitmix64.restype = C.c_uint64
        h.orc_splitmix64.argtypes = [C.c_uint64, C.c_uint64]
        h.orc_fill_i8_uniform.argtypes = [_P, C.c_int64, C.c_uint64, _I, _I]
        h.orc_fill_i8_relu_half.argtypes = [_P, C.c_int64, C.c_uint64]
        h.orc_fill_i32_uniform.argtypes = [_P, C.c_int64, C.c_uint64, _I, _I]
        h.orc_fill_f32_uniform.argtypes = [_P, C.c_int64, C.c_uint64, C.c_float, C.c_float]
        h.orc_conv_output_shape.argtypes = [_I] * 7 + [_P, _P, _P]
        h.orc_conv_qi32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P, _I, _I, _I, _P]
        h.orc_conv_i8_acc.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P, _I]
        h.orc_requant_i8.argtypes = [_P, C.c_int64, _I, _P, _P, C.c_float, C.c_float, _I, _P]
        h.orc_dequant_f32.argtypes = [_P, C.c_int64, _I, _P, _P, C.c_float, C.c_float, _I, _P]
        h.orc_bmm_i32.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I]
        h.orc_conv_f32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P, _I]
        h.orc_bprop_f32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P, _I]
        h.orc_grad_f32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P, _I]
        h.orc_block_conv_f32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P, _I, _P, _I]
        h.orc_block_bprop_f32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P, _I]
        h.orc_block_grad_f32.argtypes = [_P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I, _I, _P, _P, _I, _I]
        h.orc_block_dbias_f32.argtypes = [_P, _I, _I, _I, _I, _I, _I, _I, _I, _P]
        _orc = h
    return _orc


def ref() -> Optional[C.CDLL]:
    """The reference's compiled cpu_ref.cpp, or None where it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        h = C.CDLL(str(REF_PATH))
        h.ref_last_error.restype = C.c_char_p
        h.ref_fprop_qi32.argtypes = [C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int, _P, C.c_int, C.c_int, C.c_int,
                                     _P, _P, _I, C.c_int, C.c_int, _P, _P]
        h.ref_backward_f32.argtypes = [C.c_int, _P, _P] + [C.c_int] * 7 + [_P, _P, _P]
        h.ref_fprop_f32.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int, _P, C.c_int, C.c_int, C.c_int, _P, _P, _P]
        h.ref_block_f32.argtypes = [C.c_int, _P, _P] + [C.c_int] * 7 + [_P, C.c_int, C.c_int, _P, C.c_int, _P, _P]
        h.ref_verify_tensors.argtypes = [_P, _P, C.c_size_t, C.c_float, C.c_float, _P, _P, _P, _P, _P]
        _ref = h
    return _ref


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _conv7(conv: Sequence[int]) -> np.ndarray:
    a = np.ascontiguousarray(conv, dtype=np.int32)
    assert a.shape == (7,)
    return a


# ---- generator -------------------------------------------------------------------------

def splitmix64(seed: int, i: int) -> int:
    return int(orc().orc_splitmix64(seed, i))


def fill_i8_uniform(count, seed, lo, hi):
    out = np.empty(count, np.int8)
    orc().orc_fill_i8_uniform(_p(out), count, seed, lo, hi)
    return out


def fill_i8_relu_half(count, seed):
    out = np.empty(count, np.int8)
    orc().orc_fill_i8_relu_half(_p(out), count, seed)
    return out


def fill_i32_uniform(count, seed, lo, hi):
    out = np.empty(count, np.int32)
    orc().orc_fill_i32_uniform(_p(out), count, seed, lo, hi)
    return out


def fill_f32_uniform(count, seed, lo, hi):
    out = np.empty(count, np.float32)
    orc().orc_fill_f32_uniform(_p(out), count, seed, lo, hi)
    return out


# ---- convolution -----------------------------------------------------------------------

def conv_output_shape(n, h, w, c, r, s, k, conv) -> Optional[Tuple[int, int]]:
    ho, wo = C.c_int32(), C.c_int32()
    cv = _conv7(conv)
    if orc().orc_conv_output_shape(n, h, w, c, r, s, k, _p(cv), C.byref(ho), C.byref(wo)) != 0:
        return None
    return ho.value, wo.value


def conv_qi32(x: np.ndarray, wt: np.ndarray, conv, in_zp, f_zp: int, block=(0, 0)) -> np.ndarray:
    """int32 accumulators on float codes; x NHWC float32, wt KRSC (or K,By,Bx,R,S,C) float32."""
    x = np.ascontiguousarray(x, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, h, w, c = x.shape
    k = wt.shape[0]
    r, s = wt.shape[-3], wt.shape[-2]
    cv = _conv7(conv)
    shp = conv_output_shape(n, h, w, c, r, s, k, cv)
    if shp is None:
        raise ValueError("rejected shape")
    zp = np.ascontiguousarray(in_zp, np.int32)
    assert zp.shape == (n,)
    y = np.empty((n, shp[0], shp[1], k), np.int32)
    by, bx = block
    if orc().orc_conv_qi32(_p(x), n, h, w, c, _p(wt), r, s, k, _p(cv), _p(zp), int(f_zp), by, bx, _p(y)) != 0:
        raise ValueError("rejected shape")
    return y


def conv_i8_acc(x: np.ndarray, wt: np.ndarray, conv, nthreads: int = 0) -> np.ndarray:
    """int32 accumulators of int8 codes (zero points 0); x NHWC, wt KRSC."""
    x = np.ascontiguousarray(x, np.int8)
    wt = np.ascontiguousarray(wt, np.int8)
    n, h, w, c = x.shape
    k, r, s, _ = wt.shape
    cv = _conv7(conv)
    shp = conv_output_shape(n, h, w, c, r, s, k, cv)
    if shp is None:
        raise ValueError("rejected shape")
    y = np.empty((n, shp[0], shp[1], k), np.int32)
    if orc().orc_conv_i8_acc(_p(x), n, h, w, c, _p(wt), r, s, k, _p(cv), _p(y), nthreads) != 0:
        raise ValueError("rejected shape")
    return y


def conv_f32(x: np.ndarray, wt: np.ndarray, conv, nthreads: int = 0) -> np.ndarray:
    """fp32 convolution in the reference CPU loop's order and rounding; x NHWC, wt KRSC."""
    x = np.ascontiguousarray(x, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, h, w, c = x.shape
    k, r, s, _ = wt.shape
    cv = _conv7(conv)
    shp = conv_output_shape(n, h, w, c, r, s, k, cv)
    if shp is None:
        raise ValueError("rejected shape")
    y = np.empty((n, shp[0], shp[1], k), np.float32)
    if orc().orc_conv_f32(_p(x), n, h, w, c, _p(wt), r, s, k, _p(cv), _p(y), nthreads) != 0:
        raise ValueError("rejected shape")
    return y


def ref_conv_f32(x, wt, conv) -> Tuple[np.ndarray, float]:
    """(fp32 output, seconds) of the reference's own cpu_fprop_nhwc (oracle/_ref)."""
    h = ref()
    if h is None:
        raise RuntimeError("oracle/_ref/libref_cpu.so was not built")
    x = np.ascontiguousarray(x, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, hh, w, c = x.shape
    k, r, s, _ = wt.shape
    cv = _conv7(conv)
    shp = conv_output_shape(n, hh, w, c, r, s, k, cv)
    if shp is None:
        raise ValueError("rejected shape")
    y = np.empty((n, shp[0], shp[1], k), np.float32)
    secs = C.c_double()
    if h.ref_fprop_f32(_p(x), n, hh, w, c, _p(wt), r, s, k, _p(cv), _p(y), C.byref(secs)) != 0:
        raise RuntimeError(h.ref_last_error().decode())
    return y, secs.value


def bprop_f32(dy: np.ndarray, wt: np.ndarray, x_shape, conv, nthreads: int = 0) -> np.ndarray:
    """dx (x_shape, NHWC) of the fp32 convolution in the loop order of cpu_bprop_nhwc."""
    dy = np.ascontiguousarray(dy, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, h, w, c = (int(v) for v in x_shape)
    k, r, s, _ = wt.shape
    dx = np.empty((n, h, w, c), np.float32)
    if orc().orc_bprop_f32(_p(dy), n, h, w, c, _p(wt), r, s, k, _p(_conv7(conv)), _p(dx), nthreads) != 0:
        raise ValueError("rejected shape")
    return dx


def grad_f32(x: np.ndarray, dy: np.ndarray, w_shape, conv, nthreads: int = 0) -> np.ndarray:
    """dw (w_shape, KRSC) of the fp32 convolution in the loop order of cpu_grad_nhwc."""
    x = np.ascontiguousarray(x, np.float32)
    dy = np.ascontiguousarray(dy, np.float32)
    n, h, w, c = x.shape
    k, r, s, cg = (int(v) for v in w_shape)
    dw = np.empty((k, r, s, cg), np.float32)
    if orc().orc_grad_f32(_p(x), n, h, w, c, _p(dy), r, s, k, _p(_conv7(conv)), _p(dw), nthreads) != 0:
        raise ValueError("rejected shape")
    return dw


def ref_backward_f32(op: str, a, b, x_shape, w_shape, conv) -> Tuple[np.ndarray, float]:
    """(dx or dw, seconds) of the reference's own cpu_bprop_nhwc ('bprop': a = dy, b = w) or
    cpu_grad_nhwc ('grad': a = x, b = dy), compiled in oracle/_ref."""
    h = ref()
    if h is None:
        raise RuntimeError("oracle/_ref/libref_cpu.so was not built")
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    n, hh, w, c = (int(v) for v in x_shape)
    k, r, s, cg = (int(v) for v in w_shape)
    out = np.empty((n, hh, w, c) if op == "bprop" else (k, r, s, cg), np.float32)
    secs = C.c_double()
    if h.ref_backward_f32(0 if op == "bprop" else 1, _p(a), _p(b), n, hh, w, c, r, s, k, _p(_conv7(conv)), _p(out),
                          C.byref(secs)) != 0:
        raise RuntimeError(h.ref_last_error().decode())
    return out, secs.value


# ---- blocked fp32 ------------------------------------------------------------------------

def _bias_mode(mode) -> int:
    if mode in (0, "per_block", "PerBlock"):
        return 0
    if mode in (1, "shared", "Shared"):
        return 1
    raise ValueError(f"unknown bias mode {mode!r}")


def _block_out_shape(n, h, w, c, r, s, k, conv, by, bx):
    shp = conv_output_shape(n, h, w, c, r, s, k, _conv7(conv))
    if shp is None or by <= 0 or bx <= 0 or shp[0] % by or shp[1] % bx:
        raise ValueError("rejected shape")
    return shp


def block_conv_f32(x: np.ndarray, wt: np.ndarray, conv, bias=None, bias_mode=0, nthreads: int = 0) -> np.ndarray:
    """Blocked fp32 convolution in the loop order of cpu_block_fprop_nhwc; x NHWC, wt
    [K, By, Bx, R, S, C/groups], bias K*By*Bx floats or None."""
    x = np.ascontiguousarray(x, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, h, w, c = x.shape
    k, by, bx, r, s, _ = wt.shape
    ho, wo = _block_out_shape(n, h, w, c, r, s, k, conv, by, bx)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32).reshape(-1)
    if b is not None and b.size != k * by * bx:
        raise ValueError("bias must hold k*by*bx floats")
    y = np.empty((n, ho, wo, k), np.float32)
    if orc().orc_block_conv_f32(_p(x), n, h, w, c, _p(wt), r, s, k, _p(_conv7(conv)), by, bx, _p(b),
                                _bias_mode(bias_mode), _p(y), nthreads) != 0:
        raise ValueError("rejected shape")
    return y


def block_bprop_f32(dy: np.ndarray, wt: np.ndarray, x_shape, conv, nthreads: int = 0) -> np.ndarray:
    """dx (x_shape) of the blocked fp32 convolution in the loop order of cpu_block_bprop_nhwc."""
    dy = np.ascontiguousarray(dy, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, h, w, c = (int(v) for v in x_shape)
    k, by, bx, r, s, _ = wt.shape
    _block_out_shape(n, h, w, c, r, s, k, conv, by, bx)
    dx = np.empty((n, h, w, c), np.float32)
    if orc().orc_block_bprop_f32(_p(dy), n, h, w, c, _p(wt), r, s, k, _p(_conv7(conv)), by, bx, _p(dx),
                                 nthreads) != 0:
        raise ValueError("rejected shape")
    return dx


def block_grad_f32(x: np.ndarray, dy: np.ndarray, w_shape, conv, with_dbias=False, bias_mode=0,
                   nthreads: int = 0):
    """dw ([K, By, Bx, R, S, C/groups]) of the blocked fp32 convolution in the loop order of
    cpu_block_grad_nhwc; with with_dbias, (dw, dbias) with dbias K*By*Bx floats."""
    x = np.ascontiguousarray(x, np.float32)
    dy = np.ascontiguousarray(dy, np.float32)
    n, h, w, c = x.shape
    k, by, bx, r, s, cg = (int(v) for v in w_shape)
    _block_out_shape(n, h, w, c, r, s, k, conv, by, bx)
    dw = np.empty((k, by, bx, r, s, cg), np.float32)
    db = np.empty(k * by * bx, np.float32) if with_dbias else None
    if orc().orc_block_grad_f32(_p(x), n, h, w, c, _p(dy), r, s, k, _p(_conv7(conv)), by, bx, _p(dw), _p(db),
                                _bias_mode(bias_mode), nthreads) != 0:
        raise ValueError("rejected shape")
    return (dw, db) if with_dbias else dw


DBIAS_CHUNK = 256  # positions per run of the library's bias-gradient kernels (kDbiasChunk)


def block_dbias_f32(dy: np.ndarray, by: int, bx: int, bias_mode=0, chunk: int = DBIAS_CHUNK) -> np.ndarray:
    """The blocked bias gradient (K*By*Bx floats): dy summed over every position of each block,
    in runs of `chunk` positions added in order (chunk <= 0: one sequential run), the fixed
    order of the library's kernels for launch_block_grad_nhwc's all-positions sum."""
    dy = np.ascontiguousarray(dy, np.float32)
    n, ho, wo, k = dy.shape
    out = np.empty(k * by * bx, np.float32)
    if orc().orc_block_dbias_f32(_p(dy), n, ho, wo, k, by, bx, _bias_mode(bias_mode), chunk, _p(out)) != 0:
        raise ValueError("rejected shape")
    return out


def ref_block_f32(op: str, a, b, x_shape, w_shape, conv, bias=None, bias_mode=0):
    """(result, seconds, bias-or-dbias) of the reference's own cpu_block_fprop_nhwc ('fprop':
    a = x, b = w, bias read), cpu_block_bprop_nhwc ('bprop': a = dy, b = w) or
    cpu_block_grad_nhwc ('grad': a = x, b = dy, bias = a K*By*Bx float array that receives
    dbias, or None), compiled in oracle/_ref."""
    h = ref()
    if h is None:
        raise RuntimeError("oracle/_ref/libref_cpu.so was not built")
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    n, hh, w, c = (int(v) for v in x_shape)
    k, by, bx, r, s, cg = (int(v) for v in w_shape)
    opi = {"fprop": 0, "bprop": 1, "grad": 2}[op]
    if opi == 0:
        ho, wo = _block_out_shape(n, hh, w, c, r, s, k, conv, by, bx)
        out = np.empty((n, ho, wo, k), np.float32)
    elif opi == 1:
        out = np.empty((n, hh, w, c), np.float32)
    else:
        out = np.empty((k, by, bx, r, s, cg), np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    secs = C.c_double()
    if h.ref_block_f32(opi, _p(a), _p(b), n, hh, w, c, r, s, k, _p(_conv7(conv)), by, bx, _p(bb),
                       _bias_mode(bias_mode), _p(out), C.byref(secs)) != 0:
        raise RuntimeError(h.ref_last_error().decode())
    return out, secs.value, bb


def verify_tensors(ref_v: np.ndarray, got: np.ndarray, abs_eps: float = 1e-4, rel_eps: float = 1e-3) -> bool:
    """The pass rule of the reference's verify_tensors (src/verify.cpp:7-36): an element fails
    when |a - b| > abs_eps and (|a| <= 1e-6 or |a - b| / max(|a|, 1e-6) > rel_eps)."""
    a = np.asarray(ref_v, np.float32).ravel()
    b = np.asarray(got, np.float32).ravel()
    err = np.abs(a - b)
    rel = err / np.maximum(np.abs(a), np.float32(1e-6))
    fail = (err > abs_eps) & ((np.abs(a) <= 1e-6) | (rel > rel_eps))
    return not bool(fail.any())


def bmm_i32(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False,
            nthreads: int = 0) -> np.ndarray:
    """C[i] = op(a[i]) @ op(b[i]) with int32 wrap-around; a is (batch, M, K), or (batch, K, M)
    stored when trans_a; b is (batch, K, N), or (batch, N, K) when trans_b."""
    a = np.ascontiguousarray(a, np.int32)
    b = np.ascontiguousarray(b, np.int32)
    assert a.ndim == 3 and b.ndim == 3 and a.shape[0] == b.shape[0]
    batch = a.shape[0]
    m, k = (a.shape[2], a.shape[1]) if trans_a else (a.shape[1], a.shape[2])
    n, kb = (b.shape[1], b.shape[2]) if trans_b else (b.shape[2], b.shape[1])
    assert k == kb, (a.shape, b.shape)
    c = np.empty((batch, m, n), np.int32)
    orc().orc_bmm_i32(_p(a), _p(b), _p(c), batch, m, n, k, int(bool(trans_a)), int(bool(trans_b)), nthreads)
    return c


def requant_i8(acc: np.ndarray, bias, w_scale, in_scale, out_scale, relu) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.int32)
    k = acc.shape[-1]
    b = None if bias is None else np.ascontiguousarray(bias, np.int32)
    ws = np.ascontiguousarray(w_scale, np.float32)
    y = np.empty(acc.shape, np.int8)
    orc().orc_requant_i8(_p(acc), acc.size // k, k, _p(b), _p(ws), in_scale, out_scale, 1 if relu else 0, _p(y))
    return y


def dequant_f32(acc: np.ndarray, bias, w_scale, in_scale, out_scale, relu) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.int32)
    k = acc.shape[-1]
    b = None if bias is None else np.ascontiguousarray(bias, np.int32)
    ws = np.ascontiguousarray(w_scale, np.float32)
    y = np.empty(acc.shape, np.float32)
    orc().orc_dequant_f32(_p(acc), acc.size // k, k, _p(b), _p(ws), in_scale, out_scale, 1 if relu else 0, _p(y))
    return y


# ---- the reference's own CPU path --------------------------------------------------------

def ref_conv_qi32(kind: str, x, wt, conv, in_zp, f_zp, block=(0, 0)) -> Tuple[np.ndarray, float]:
    """(int32 output, seconds) of the reference's cpu_(block_)fprop_nhwc_qi32<kind>."""
    h = ref()
    if h is None:
        raise RuntimeError("oracle/_ref/libref_cpu.so was not built")
    x = np.ascontiguousarray(x, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    n, hh, w, c = x.shape
    k = wt.shape[0]
    r, s = wt.shape[-3], wt.shape[-2]
    cv = _conv7(conv)
    shp = conv_output_shape(n, hh, w, c, r, s, k, cv)
    if shp is None:
        raise ValueError("rejected shape")
    y = np.empty((n, shp[0], shp[1], k), np.int32)
    zp = np.ascontiguousarray(in_zp, np.int32)
    secs = C.c_double()
    st = h.ref_fprop_qi32(0 if kind == "u8" else 1, _p(x), n, hh, w, c, _p(wt), r, s, k, _p(cv), _p(zp), int(f_zp),
                          block[0], block[1], _p(y), C.byref(secs))
    if st != 0:
        raise RuntimeError(h.ref_last_error().decode())
    return y, secs.value


def ref_verify_tensors(refv, got, abs_eps, rel_eps) -> dict:
    h = ref()
    if h is None:
        raise RuntimeError("oracle/_ref/libref_cpu.so was not built")
    a = np.ascontiguousarray(refv, np.float32)
    b = np.ascontiguousarray(got, np.float32)
    ma, mr = C.c_float(), C.c_float()
    ia, ir = C.c_size_t(), C.c_size_t()
    ok = C.c_int()
    if h.ref_verify_tensors(_p(a), _p(b), a.size, abs_eps, rel_eps, C.byref(ma), C.byref(mr), C.byref(ia),
                            C.byref(ir), C.byref(ok)) != 0:
        raise RuntimeError(h.ref_last_error().decode())
    return {"max_abs_err": ma.value, "max_rel_err": mr.value, "max_abs_idx": ia.value, "max_rel_idx": ir.value,
            "passed": bool(ok.value)}
