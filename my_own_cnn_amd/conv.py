"""Python mirror of the quantized-convolution interface, over libmiq_qconv's C-ABI.

Names, argument order and error behaviour follow the reference's C++ surface
(/root/reference/src/conv_types.h:125-169, :255-340): shape inference raises with the
reference's messages, a missing quantization parameter raises before anything runs, and
every launch is asynchronous on the given (default: PyTorch's current) HIP stream.

Device tensors are ``torch`` tensors on a ROCm device (PyTorch is used only to own device
memory and streams) or raw integer device addresses.
"""
from __future__ import annotations

import ctypes as C
import enum
from typing import Optional, Sequence, Tuple, Union

import numpy as np

from . import _capi
from ._capi import (ALGO_NAMES, ALGOS, F32_KERNEL_NAMES, BlockConv2DParams, Conv2DParams, MiqError, QConvDesc, QParamsS5,
                    QParamsU8, check, lib)

try:
    import torch
except ImportError:  # pragma: no cover
    torch = None

Pointer = Union[int, "torch.Tensor", None]


class DataType(enum.IntEnum):
    """Mirror of nnalgebra::DataType (nnalgebra_quantization.h:19-24, plus LinQuantI8)."""

    Real32 = 0
    LinQuantU8 = 1
    LinQuantS5 = 2
    LinQuantI32 = 3
    LinQuantI8 = 4


SUPPORTED_QI32_INPUTS = (DataType.LinQuantU8, DataType.LinQuantS5)

# numpy views of the raw parameter structs, for building the device arrays in_qp / f_qp
QPARAMS_U8_DTYPE = np.dtype({"names": ["zero_point", "scale", "symmetric"],
                             "formats": [np.uint8, np.float32, np.uint8], "offsets": [0, 4, 8], "itemsize": 12})
QPARAMS_S5_DTYPE = np.dtype({"names": ["zero_point", "n_bins", "scale"],
                             "formats": [np.int8, np.uint8, np.float32], "offsets": [0, 1, 4], "itemsize": 8})


def qparams_array(tin: DataType, zero_points: Sequence[int], scales: Optional[Sequence[float]] = None,
                  n_bins: int = 0, symmetric: bool = False) -> np.ndarray:
    """Host array of QuantizationParameters<tin> structs with the reference's byte layout."""
    tin = DataType(tin)
    count = len(zero_points)
    scales = [1.0] * count if scales is None else list(scales)
    if tin == DataType.LinQuantU8:
        a = np.zeros(count, dtype=QPARAMS_U8_DTYPE)
        a["zero_point"] = np.asarray(zero_points, dtype=np.int64).astype(np.uint8)
        a["scale"] = scales
        a["symmetric"] = 1 if symmetric else 0
    elif tin == DataType.LinQuantS5:
        a = np.zeros(count, dtype=QPARAMS_S5_DTYPE)
        a["zero_point"] = np.asarray(zero_points, dtype=np.int64).astype(np.int8)
        a["n_bins"] = n_bins
        a["scale"] = scales
    else:
        raise ValueError("quantized int32 convolution supports only LinQuantU8 and LinQuantS5")
    return a


def _addr(t: Pointer) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise ValueError("tensor arguments must live in device memory")
    if not t.is_contiguous():
        raise ValueError("tensor arguments must be contiguous")
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        if torch is None:
            return None
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _as_params(p) -> Conv2DParams:
    if p is None:
        return Conv2DParams()
    if isinstance(p, Conv2DParams):
        return p
    return Conv2DParams(*p)


def _pair(v) -> Tuple[int, int]:
    return (v, v) if isinstance(v, int) else (int(v[0]), int(v[1]))


# ---- shape inference ---------------------------------------------------------------------

def infer_conv_shape(n: int, h: int, w: int, c: int, r: int, s: int, k: int, p=None) -> Tuple[int, int]:
    """(Ho, Wo); raises MiqError with infer_conv_shape's message on a rejected shape."""
    ho, wo = C.c_int32(), C.c_int32()
    params = _as_params(p)
    check(lib().miq_conv2d_output_shape(n, h, w, c, r, s, k, C.byref(params), C.byref(ho), C.byref(wo)),
          "infer_conv_shape")
    return ho.value, wo.value


def infer_block_conv_shape(n, h, w, c, r, s, k, p: BlockConv2DParams) -> Tuple[int, int, int, int]:
    """(Ho, Wo, block_ho, block_wo) with infer_block_conv_shape's rules."""
    out = [C.c_int32() for _ in range(4)]
    check(lib().miq_block_conv2d_output_shape(n, h, w, c, r, s, k, C.byref(p), *[C.byref(o) for o in out]),
          "infer_block_conv_shape")
    return tuple(o.value for o in out)


# ---- reference-compatible int32 accumulator path ------------------------------------------

def launch_fprop_nhwc_qi32(tin: DataType, d_x: Pointer, d_w: Pointer, d_y: Pointer, n: int, h: int, w: int, c: int,
                           r: int, s: int, k: int, p=None, in_qp: Pointer = None, f_qp: Pointer = None,
                           stream=None) -> None:
    """Mirror of launch_fprop_nhwc_qi32<Tin> (conv_types.h:308-323)."""
    tin = DataType(tin)
    if tin not in SUPPORTED_QI32_INPUTS:
        raise TypeError("launch_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5")
    if in_qp is None or f_qp is None:
        raise RuntimeError("quantized CUDA fprop requires non-null quantization parameters")
    fn = lib().miq_fprop_nhwc_qi32_u8 if tin == DataType.LinQuantU8 else lib().miq_fprop_nhwc_qi32_s5
    params = _as_params(p)
    check(fn(_addr(d_x), _addr(d_w), _addr(d_y), n, h, w, c, r, s, k, C.byref(params), _addr(in_qp), _addr(f_qp),
             _stream(stream)), "launch_fprop_nhwc_qi32")


QI32_ALGOS = {"auto": 0, "direct": 1, "igemm": 2, "band": 4, "stream": 5, "stem_s2d": 11}


def fprop_nhwc_qi32_algo(tin: DataType, d_x: Pointer, d_w: Pointer, d_y: Pointer, n: int, h: int, w: int, c: int,
                         r: int, s: int, k: int, p=None, in_qp: Pointer = None, f_qp: Pointer = None,
                         algo: str = "auto", stream=None, workspace: Pointer = None, workspace_bytes: int = 0) -> None:
    """launch_fprop_nhwc_qi32 with an explicit kernel ("auto", "band", "stream", "stem_s2d",
    "igemm" or "direct"); every choice gives the same int32 results.  `workspace`: a device buffer of at
    least qi32_workspace_size() bytes, which makes the call allocation-free
    (miq_fprop_nhwc_qi32_ws); None uses the library's per-stream workspace."""
    tin = DataType(tin)
    if tin not in SUPPORTED_QI32_INPUTS:
        raise TypeError("launch_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5")
    if in_qp is None or f_qp is None:
        raise RuntimeError("quantized CUDA fprop requires non-null quantization parameters")
    params = _as_params(p)
    kind = 0 if tin == DataType.LinQuantU8 else 1
    if workspace is None:
        check(lib().miq_fprop_nhwc_qi32_algo(kind, _addr(d_x), _addr(d_w), _addr(d_y), n, h, w, c, r, s, k,
                                             C.byref(params), _addr(in_qp), _addr(f_qp), QI32_ALGOS[algo],
                                             _stream(stream)), "fprop_nhwc_qi32_algo")
    else:
        check(lib().miq_fprop_nhwc_qi32_ws(kind, _addr(d_x), _addr(d_w), _addr(d_y), n, h, w, c, r, s, k,
                                           C.byref(params), _addr(in_qp), _addr(f_qp), QI32_ALGOS[algo],
                                           _addr(workspace), workspace_bytes, _stream(stream)), "fprop_nhwc_qi32_ws")


def qi32_workspace_size(n: int, h: int, w: int, c: int, r: int, s: int, k: int, p=None, algo: str = "auto") -> int:
    """Bytes of device workspace fprop_nhwc_qi32_algo(..., workspace=...) needs (no GPU access)."""
    out = C.c_size_t()
    params = _as_params(p)
    check(lib().miq_fprop_nhwc_qi32_workspace_size(n, h, w, c, r, s, k, C.byref(params), QI32_ALGOS[algo],
                                                   C.byref(out)), "qi32_workspace_size")
    return out.value


def plan_qi32(n: int, h: int, w: int, c: int, r: int, s: int, k: int, p=None) -> str:
    """The kernel launch_fprop_nhwc_qi32 runs for this problem (aligned tensors)."""
    out = C.c_int32()
    params = _as_params(p)
    check(lib().miq_plan_qi32(n, h, w, c, r, s, k, C.byref(params), C.byref(out)), "plan_qi32")
    return {v: key for key, v in QI32_ALGOS.items()}[out.value]


def plan_block_qi32(n: int, h: int, w: int, c: int, r: int, s: int, k: int, p: BlockConv2DParams) -> str:
    """The kernel launch_block_fprop_nhwc_qi32 runs for this problem (aligned tensors)."""
    out = C.c_int32()
    check(lib().miq_plan_block_qi32(n, h, w, c, r, s, k, C.byref(p), C.byref(out)), "plan_block_qi32")
    return {v: key for key, v in QI32_ALGOS.items()}[out.value]


def launch_block_fprop_nhwc_qi32(tin: DataType, d_x: Pointer, d_w: Pointer, d_y: Pointer, n: int, h: int, w: int,
                                 c: int, r: int, s: int, k: int, p: BlockConv2DParams, in_qp: Pointer = None,
                                 f_qp: Pointer = None, stream=None) -> None:
    """Mirror of launch_block_fprop_nhwc_qi32<Tin> (conv_types.h:325-340)."""
    tin = DataType(tin)
    if tin not in SUPPORTED_QI32_INPUTS:
        raise TypeError("launch_block_fprop_nhwc_qi32 supports only LinQuantU8 and LinQuantS5")
    if in_qp is None or f_qp is None:
        raise RuntimeError("quantized blocked CUDA fprop requires non-null quantization parameters")
    fn = lib().miq_block_fprop_nhwc_qi32_u8 if tin == DataType.LinQuantU8 else lib().miq_block_fprop_nhwc_qi32_s5
    check(fn(_addr(d_x), _addr(d_w), _addr(d_y), n, h, w, c, r, s, k, C.byref(p), _addr(in_qp), _addr(f_qp),
             _stream(stream)), "launch_block_fprop_nhwc_qi32")


# ---- native int8 path -------------------------------------------------------------------

def make_desc(x_shape, w_shape, *, stride=1, padding=0, dilation=1, groups=1, relu=False, in_scale=1.0,
              out_scale=1.0, algo="auto") -> QConvDesc:
    """Descriptor for x NHWC and w KRSC shapes."""
    n, h, w, c = (int(v) for v in x_shape)
    k, r, s, _ = (int(v) for v in w_shape)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    d = QConvDesc()
    d.n, d.h, d.w, d.c = n, h, w, c
    d.k, d.r, d.s = k, r, s
    d.conv = Conv2DParams(ph, pw, sh, sw, dh, dw, groups)
    d.relu = 1 if relu else 0
    d.in_scale = float(in_scale)
    d.out_scale = float(out_scale)
    d.algo = ALGOS[algo] if isinstance(algo, str) else int(algo)
    return d


def plan(desc: QConvDesc) -> str:
    """Kernel family ('flat', 'band', 'stream', 'igemm', 'stem' or 'direct') the int8 entry points will run."""
    a = C.c_int32()
    check(lib().miq_qconv2d_plan(C.byref(desc), C.byref(a)), "plan")
    return ALGO_NAMES[a.value]


def _out(x, w, desc: QConvDesc, dtype, out):
    ho, wo = infer_conv_shape(desc.n, desc.h, desc.w, desc.c, desc.r, desc.s, desc.k, desc.conv)
    shape = (desc.n, ho, wo, desc.k)
    if out is None:
        return torch.empty(shape, dtype=dtype, device=x.device)
    if tuple(out.shape) != shape or out.dtype != dtype:
        raise ValueError(f"out must be {dtype} of shape {shape}")
    return out


def qconv2d_nhwc_i8(x, w, bias, w_scale, *, stride=1, padding=0, dilation=1, groups=1, relu=False,
                    in_scale=1.0, out_scale=1.0, algo="auto", out=None, stream=None):
    """int8 NHWC output of conv + bias + per-channel requantize (+ ReLU) + saturate."""
    desc = make_desc(x.shape, w.shape, stride=stride, padding=padding, dilation=dilation, groups=groups,
                     relu=relu, in_scale=in_scale, out_scale=out_scale, algo=algo)
    y = _out(x, w, desc, torch.int8, out)
    check(lib().miq_qconv2d_nhwc_i8(C.byref(desc), _addr(x), _addr(w), _addr(bias), _addr(w_scale), _addr(y),
                                    _stream(stream)), "qconv2d_nhwc_i8")
    return y


def qconv2d_nhwc_i8_acc32(x, w, *, stride=1, padding=0, dilation=1, groups=1, algo="auto", out=None,
                          stream=None):
    """Raw int32 accumulators of the int8 convolution."""
    desc = make_desc(x.shape, w.shape, stride=stride, padding=padding, dilation=dilation, groups=groups, algo=algo)
    y = _out(x, w, desc, torch.int32, out)
    check(lib().miq_qconv2d_nhwc_i8_acc32(C.byref(desc), _addr(x), _addr(w), _addr(y), _stream(stream)),
          "qconv2d_nhwc_i8_acc32")
    return y


def qconv2d_nhwc_i8_dequant(x, w, bias, w_scale, *, stride=1, padding=0, dilation=1, groups=1, relu=False,
                            in_scale=1.0, out_scale=1.0, algo="auto", out=None, stream=None):
    """fp32 dequantized view (float(acc + bias) * multiplier, optional ReLU)."""
    desc = make_desc(x.shape, w.shape, stride=stride, padding=padding, dilation=dilation, groups=groups,
                     relu=relu, in_scale=in_scale, out_scale=out_scale, algo=algo)
    y = _out(x, w, desc, torch.float32, out)
    check(lib().miq_qconv2d_nhwc_i8_dequant(C.byref(desc), _addr(x), _addr(w), _addr(bias), _addr(w_scale),
                                            _addr(y), _stream(stream)), "qconv2d_nhwc_i8_dequant")
    return y



F32_ALGOS = {"auto": 0, "direct": 1, "igemm": 2}
F32_GRAD_ALGOS = {"auto": 0, "direct": 1, "igemm": 2, "atomic": 6}


def launch_fprop_nhwc(d_x: Pointer, d_w: Pointer, d_y: Pointer, n: int, h: int, w: int, c: int, r: int, s: int,
                      k: int, p=None, algo: str = "auto", stream=None) -> None:
    """Mirror of launch_fprop_nhwc (conv_types.h:287-289, cuda_kernels.cu:767-823): fp32 NHWC
    convolution on device pointers; `algo` 'auto', 'igemm' (MFMA) or 'direct'."""
    params = _as_params(p)
    check(lib().miq_fprop_nhwc_f32(_addr(d_x), _addr(d_w), _addr(d_y), n, h, w, c, r, s, k, C.byref(params),
                                   F32_ALGOS[algo], _stream(stream)), "launch_fprop_nhwc")



def launch_bprop_nhwc(d_dy: Pointer, d_w: Pointer, d_dx: Pointer, n: int, h: int, w: int, c: int, r: int, s: int,
                      k: int, p=None, algo: str = "auto", stream=None) -> None:
    """Mirror of launch_bprop_nhwc (conv_types.h:290-292): dx of the fp32 convolution; `algo`
    'auto', 'igemm' (MFMA, stride 1) or 'direct' (bit-exact with cpu_bprop_nhwc)."""
    params = _as_params(p)
    check(lib().miq_bprop_nhwc_f32(_addr(d_dy), _addr(d_w), _addr(d_dx), n, h, w, c, r, s, k, C.byref(params),
                                   F32_ALGOS[algo], _stream(stream)), "launch_bprop_nhwc")


def launch_grad_nhwc(d_x: Pointer, d_dy: Pointer, d_dw: Pointer, n: int, h: int, w: int, c: int, r: int, s: int,
                     k: int, p=None, algo: str = "auto", stream=None, workspace=None) -> None:
    """Mirror of launch_grad_nhwc (conv_types.h:293-295): dw of the fp32 convolution; `algo`
    'auto' / 'igemm' (split over pixels, partial sums added in a fixed order: the same bits on
    every call), 'atomic' (float-atomic partial sums, no workspace) or 'direct' (bit-exact with
    cpu_grad_nhwc).  `workspace`: a device buffer of at least grad_workspace_size() bytes,
    which makes the call allocation-free (miq_grad_nhwc_f32_ws); None uses the library's
    cached per-device workspace."""
    params = _as_params(p)
    a = F32_GRAD_ALGOS[algo]
    if workspace is None:
        check(lib().miq_grad_nhwc_f32(_addr(d_x), _addr(d_dy), _addr(d_dw), n, h, w, c, r, s, k, C.byref(params), a,
                                      _stream(stream)), "launch_grad_nhwc")
        return
    nbytes = workspace.numel() * workspace.element_size() if hasattr(workspace, "numel") else int(workspace[1])
    ptr = _addr(workspace) if hasattr(workspace, "numel") else workspace[0]
    check(lib().miq_grad_nhwc_f32_ws(_addr(d_x), _addr(d_dy), _addr(d_dw), n, h, w, c, r, s, k, C.byref(params), a,
                                     ptr, nbytes, _stream(stream)), "launch_grad_nhwc")


def grad_workspace_size(n: int, h: int, w: int, c: int, r: int, s: int, k: int, p=None, algo: str = "auto") -> int:
    """Bytes of device workspace launch_grad_nhwc(..., workspace=...) needs (no GPU access)."""
    params = _as_params(p)
    out = C.c_size_t(0)
    check(lib().miq_grad_nhwc_f32_workspace_size(n, h, w, c, r, s, k, C.byref(params), F32_GRAD_ALGOS[algo],
                                                 C.byref(out)), "grad_workspace_size")
    return int(out.value)

def plan_f32(op: str, n: int, h: int, w: int, c: int, r: int, s: int, k: int, p=None, algo: str = "auto") -> str:
    """Kernel family an fp32 pass ('fprop', 'bprop' or 'grad') runs for this problem with aligned
    tensors: the library's own dispatch (miq_plan_f32), no GPU access."""
    params = _as_params(p)
    ops = {"fprop": 0, "bprop": 1, "grad": 2}
    algos = F32_GRAD_ALGOS if op == "grad" else F32_ALGOS
    if op not in ops:
        raise ValueError(f"op must be one of {sorted(ops)}, got {op!r}")
    if algo not in algos:
        raise ValueError(f"algo for {op} must be one of {sorted(algos)}, got {algo!r}")
    out = C.c_int32()
    check(lib().miq_plan_f32(ops[op], n, h, w, c, r, s, k, C.byref(params), algos[algo], C.byref(out)), "plan_f32")
    return F32_KERNEL_NAMES[out.value]


BLOCK_BIAS_MODES = {"per_block": 0, "shared": 1}


def _bias_mode(mode) -> int:
    if isinstance(mode, str):
        if mode not in BLOCK_BIAS_MODES:
            raise ValueError(f"bias_mode must be one of {sorted(BLOCK_BIAS_MODES)}, got {mode!r}")
        return BLOCK_BIAS_MODES[mode]
    return int(mode)


def _check_algo(algo: str, algos) -> int:
    if algo not in algos:
        raise ValueError(f"algo must be one of {sorted(algos)}, got {algo!r}")
    return algos[algo]


def launch_block_fprop_nhwc(d_x: Pointer, d_w: Pointer, d_y: Pointer, n: int, h: int, w: int, c: int, r: int,
                            s: int, k: int, p: BlockConv2DParams, d_bias: Pointer = None, bias_mode="per_block",
                            algo: str = "auto", stream=None) -> None:
    """Mirror of launch_block_fprop_nhwc (conv_types.h:296-299, cuda_kernels.cu:939-1001): the
    blocked fp32 convolution, filter [K, By, Bx, R, S, C/groups], optional bias [K, By, Bx]
    (bias_mode 'per_block' or 'shared'); `algo` 'auto', 'igemm' (MFMA) or 'direct' (bit-exact
    with cpu_block_fprop_nhwc)."""
    check(lib().miq_block_fprop_nhwc_f32(_addr(d_x), _addr(d_w), _addr(d_y), n, h, w, c, r, s, k, C.byref(p),
                                         _addr(d_bias), _bias_mode(bias_mode), _check_algo(algo, F32_ALGOS),
                                         _stream(stream)), "launch_block_fprop_nhwc")


def launch_block_bprop_nhwc(d_dy: Pointer, d_w: Pointer, d_dx: Pointer, n: int, h: int, w: int, c: int, r: int,
                            s: int, k: int, p: BlockConv2DParams, algo: str = "auto", stream=None) -> None:
    """Mirror of launch_block_bprop_nhwc (conv_types.h:300-302, cuda_kernels.cu:1003-1058): dx of
    the blocked fp32 convolution; `algo` 'auto', 'igemm' (MFMA, stride 1) or 'direct' (bit-exact
    with cpu_block_bprop_nhwc)."""
    check(lib().miq_block_bprop_nhwc_f32(_addr(d_dy), _addr(d_w), _addr(d_dx), n, h, w, c, r, s, k, C.byref(p),
                                         _check_algo(algo, F32_ALGOS), _stream(stream)), "launch_block_bprop_nhwc")


def launch_block_grad_nhwc(d_x: Pointer, d_dy: Pointer, d_dw: Pointer, n: int, h: int, w: int, c: int, r: int,
                           s: int, k: int, p: BlockConv2DParams, d_dbias: Pointer = None, bias_mode="per_block",
                           algo: str = "auto", stream=None) -> None:
    """Mirror of launch_block_grad_nhwc (conv_types.h:303-305, cuda_kernels.cu:1060-1136): dw of
    the blocked fp32 convolution and, with d_dbias, the bias gradient (the sum of dy over every
    position of each block, in a fixed order); `algo` as launch_grad_nhwc ('direct' gives
    cpu_block_grad_nhwc's dw bit for bit)."""
    check(lib().miq_block_grad_nhwc_f32(_addr(d_x), _addr(d_dy), _addr(d_dw), n, h, w, c, r, s, k, C.byref(p),
                                        _addr(d_dbias), _bias_mode(bias_mode), _check_algo(algo, F32_GRAD_ALGOS),
                                        _stream(stream)), "launch_block_grad_nhwc")


def plan_block_f32(op: str, n: int, h: int, w: int, c: int, r: int, s: int, k: int, p: BlockConv2DParams,
                   algo: str = "auto") -> str:
    """plan_f32 for the blocked passes (miq_plan_block_f32), no GPU access."""
    ops = {"fprop": 0, "bprop": 1, "grad": 2}
    if op not in ops:
        raise ValueError(f"op must be one of {sorted(ops)}, got {op!r}")
    a = _check_algo(algo, F32_GRAD_ALGOS if op == "grad" else F32_ALGOS)
    out = C.c_int32()
    check(lib().miq_plan_block_f32(ops[op], n, h, w, c, r, s, k, C.byref(p), a, C.byref(out)), "plan_block_f32")
    return F32_KERNEL_NAMES[out.value]


def conv2d_nhwc_f32(x, w, *, stride=1, padding=0, dilation=1, groups=1, algo="auto", out=None, stream=None):
    """fp32 convolution of device tensors: x (N, H, W, C), w (K, R, S, C/groups) -> (N, Ho, Wo, K)."""
    if x.dtype != torch.float32 or w.dtype != torch.float32:
        raise ValueError("conv2d_nhwc_f32 operands must be float32")
    n, h, wd, c = (int(v) for v in x.shape)
    k, r, s = int(w.shape[0]), int(w.shape[1]), int(w.shape[2])
    (sh, sw), (ph, pw), (dh, dw) = _pair(stride), _pair(padding), _pair(dilation)
    params = Conv2DParams(ph, pw, sh, sw, dh, dw, groups)
    ho, wo = infer_conv_shape(n, h, wd, c, r, s, k, params)
    if out is None:
        out = torch.empty((n, ho, wo, k), dtype=torch.float32, device=x.device)
    elif tuple(out.shape) != (n, ho, wo, k) or out.dtype != torch.float32:
        raise ValueError(f"out must be float32 of shape {(n, ho, wo, k)}")
    launch_fprop_nhwc(x, w, out, n, h, wd, c, r, s, k, params, algo, stream)
    return out

def bmm_matmul_i32(d_A: Pointer, d_B: Pointer, d_C: Pointer, batch: int, M: int, N: int, K: int, trans_a: int,
                   trans_b: int, stream=None) -> None:
    """bmm_matmul_i32 (/root/reference/bmm.cu:298-322) on device pointers: C[b] = op(A[b]) op(B[b])
    with int32 wrap-around, A[b] M x K (stored K x M when trans_a), B[b] K x N (stored N x K
    when trans_b).  Raises MiqError where the C symbol would record an error and return."""
    check(lib().miq_bmm_i32(_addr(d_A), _addr(d_B), _addr(d_C), batch, M, N, K, 1 if trans_a else 0,
                            1 if trans_b else 0, _stream(stream)), "bmm_matmul_i32")


def bmm_i32(a, b, *, trans_a=False, trans_b=False, out=None, stream=None):
    """int32 batched product of device tensors: a (batch, M, K), or (batch, K, M) when
    trans_a; b (batch, K, N), or (batch, N, K) when trans_b; 2-D operands are one batch
    entry.  Returns (batch, M, N) int32 (2-D when both operands were)."""
    if a.dtype != torch.int32 or b.dtype != torch.int32:
        raise ValueError("bmm_i32 operands must be int32")
    two_d = a.dim() == 2 and b.dim() == 2
    a3 = a.unsqueeze(0) if a.dim() == 2 else a
    b3 = b.unsqueeze(0) if b.dim() == 2 else b
    if a3.dim() != 3 or b3.dim() != 3 or a3.shape[0] != b3.shape[0]:
        raise ValueError(f"bmm_i32 operands must be 3-D with equal batch, got {tuple(a.shape)} and {tuple(b.shape)}")
    batch = a3.shape[0]
    m, k = (a3.shape[2], a3.shape[1]) if trans_a else (a3.shape[1], a3.shape[2])
    n, kb = (b3.shape[1], b3.shape[2]) if trans_b else (b3.shape[2], b3.shape[1])
    if k != kb:
        raise ValueError(f"bmm_i32 inner extents differ: {k} and {kb}")
    shape = (batch, m, n)
    if out is None:
        y = torch.empty(shape, dtype=torch.int32, device=a.device)
    else:
        if tuple(out.shape) not in (shape, shape[1:]) or out.dtype != torch.int32:
            raise ValueError(f"out must be int32 of shape {shape}")
        y = out
    bmm_matmul_i32(a3, b3, y, batch, m, n, k, trans_a, trans_b, stream)
    return y[0] if two_d and out is None else y

__all__ = [
    "bmm_i32", "bmm_matmul_i32", "conv2d_nhwc_f32", "launch_fprop_nhwc", "launch_bprop_nhwc", "launch_grad_nhwc",
    "launch_block_fprop_nhwc", "launch_block_bprop_nhwc", "launch_block_grad_nhwc", "plan_block_f32",
    "DataType", "Conv2DParams", "BlockConv2DParams", "QParamsU8", "QParamsS5", "QConvDesc", "MiqError",
    "qparams_array", "infer_conv_shape", "infer_block_conv_shape", "launch_fprop_nhwc_qi32",
    "launch_block_fprop_nhwc_qi32", "make_desc", "plan", "plan_f32", "qconv2d_nhwc_i8", "qconv2d_nhwc_i8_acc32",
    "qconv2d_nhwc_i8_dequant",
]
_ = _capi
