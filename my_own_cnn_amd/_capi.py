"""ctypes declarations of libmiq_qconv's C-ABI (include/miq_qconv.h).

The library must be built in-tree (``python -m my_own_cnn_amd.build``).  Loading fails
loudly when it is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

# PyTorch ships its own HIP runtime under the same SONAME (libamdhip64.so.7).  Importing
# torch first makes the dynamic loader bind libmiq_qconv to that one copy, so device
# pointers and streams created by torch are valid in the library.
try:  # pragma: no cover - import side effect only
    import torch  # noqa: F401
except ImportError:  # the C-ABI itself does not need torch
    torch = None

LIB_PATH = Path(__file__).resolve().parent / "libmiq_qconv.so"

MIQ_OK = 0
MIQ_ERR_NULL_POINTER = 1
MIQ_ERR_INVALID_ARGUMENT = 2
MIQ_ERR_UNSUPPORTED = 3
MIQ_ERR_HIP = 4

MIQ_ALGO_AUTO = 0
MIQ_ALGO_DIRECT = 1
MIQ_ALGO_IGEMM = 2
MIQ_ALGO_STEM = 3
MIQ_ALGO_BAND = 4
MIQ_ALGO_STREAM = 5
MIQ_ALGO_ATOMIC = 6  # fp32 grad only
MIQ_ALGO_FLAT = 7
MIQ_ALGO_DOT4 = 8
MIQ_ALGO_PIPE = 9
MIQ_ALGO_POINTWISE = 10
MIQ_ALGO_STEM_S2D = 11

# miq_f32_kernel: the fp32 passes' kernel families (miq_plan_f32)
F32_KERNEL_NAMES = {0: "direct", 1: "igemm", 2: "igemm32", 3: "depthwise", 4: "bprop_igemm", 5: "grad_igemm",
                    6: "grad_depthwise"}
ALGOS = {"auto": MIQ_ALGO_AUTO, "direct": MIQ_ALGO_DIRECT, "igemm": MIQ_ALGO_IGEMM, "stem": MIQ_ALGO_STEM,
         "band": MIQ_ALGO_BAND, "stream": MIQ_ALGO_STREAM, "flat": MIQ_ALGO_FLAT, "dot4": MIQ_ALGO_DOT4,
         "pipe": MIQ_ALGO_PIPE, "pointwise": MIQ_ALGO_POINTWISE,
         "stem_s2d": MIQ_ALGO_STEM_S2D}
ALGO_NAMES = {v: k for k, v in ALGOS.items()}


class Conv2DParams(C.Structure):
    """Same fields and defaults as the reference's Conv2DParams (conv_types.h:21-29)."""

    _fields_ = [
        ("pad_h", C.c_int32),
        ("pad_w", C.c_int32),
        ("stride_h", C.c_int32),
        ("stride_w", C.c_int32),
        ("dilation_h", C.c_int32),
        ("dilation_w", C.c_int32),
        ("groups", C.c_int32),
    ]

    def __init__(self, pad_h=1, pad_w=1, stride_h=1, stride_w=1, dilation_h=1, dilation_w=1, groups=1):
        super().__init__(pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, groups)

    def as_tuple(self):
        return (self.pad_h, self.pad_w, self.stride_h, self.stride_w, self.dilation_h, self.dilation_w, self.groups)


class BlockConv2DParams(C.Structure):
    """Same layout as the reference's BlockConv2DParams (conv_types.h:31-35)."""

    _fields_ = [("conv", Conv2DParams), ("block_by", C.c_int32), ("block_bx", C.c_int32)]

    def __init__(self, conv=None, block_by=1, block_bx=1):
        super().__init__(conv if conv is not None else Conv2DParams(), block_by, block_bx)


class QParamsU8(C.Structure):
    """Byte layout of QuantizationParameters<LinQuantU8> (12 bytes)."""

    _fields_ = [("zero_point", C.c_uint8), ("scale", C.c_float), ("symmetric", C.c_uint8)]


class QParamsS5(C.Structure):
    """Byte layout of QuantizationParameters<LinQuantS5> (8 bytes)."""

    _fields_ = [("zero_point", C.c_int8), ("n_bins", C.c_uint8), ("scale", C.c_float)]


class QConvDesc(C.Structure):
    _fields_ = [
        ("n", C.c_int32), ("h", C.c_int32), ("w", C.c_int32), ("c", C.c_int32),
        ("k", C.c_int32), ("r", C.c_int32), ("s", C.c_int32),
        ("conv", Conv2DParams),
        ("relu", C.c_int32),
        ("in_scale", C.c_float),
        ("out_scale", C.c_float),
        ("algo", C.c_int32),
    ]


assert C.sizeof(Conv2DParams) == 28 and C.sizeof(BlockConv2DParams) == 36
assert C.sizeof(QParamsU8) == 12 and C.sizeof(QParamsS5) == 8

_P = C.c_void_p
_I = C.c_int32
_PI = C.POINTER(C.c_int32)

# name -> (restype, argtypes); every function declared in include/miq_qconv.h
SIGNATURES = {
    "miq_version": (C.c_int, []),
    "miq_status_string": (C.c_char_p, [C.c_int]),
    "miq_last_error_message": (C.c_char_p, []),
    "miq_conv2d_output_shape": (C.c_int, [_I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _PI, _PI]),
    "miq_block_conv2d_output_shape": (
        C.c_int, [_I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _PI, _PI, _PI, _PI]),
    "miq_qconv2d_plan": (C.c_int, [C.POINTER(QConvDesc), _PI]),
    "miq_plan_f32": (C.c_int, [_I, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, _PI]),
    "miq_fprop_nhwc_qi32_u8": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _P, _P, _P]),
    "miq_fprop_nhwc_qi32_s5": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _P, _P, _P]),
    "miq_block_fprop_nhwc_qi32_u8": (
        C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _P, _P, _P]),
    "miq_block_fprop_nhwc_qi32_s5": (
        C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _P, _P, _P]),
    "miq_fprop_nhwc_qi32_algo": (
        C.c_int, [_I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _P, _P, _I, _P]),
    "miq_plan_qi32": (C.c_int, [_I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _PI]),
    "miq_plan_block_qi32": (C.c_int, [_I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _PI]),
    "miq_fprop_nhwc_qi32_workspace_size": (
        C.c_int, [_I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, C.POINTER(C.c_size_t)]),
    "miq_fprop_nhwc_qi32_ws": (
        C.c_int, [_I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _P, _P, _I, _P, C.c_size_t,
                  _P]),
    "miq_qconv2d_nhwc_i8": (C.c_int, [C.POINTER(QConvDesc), _P, _P, _P, _P, _P, _P]),
    "miq_qconv2d_nhwc_i8_acc32": (C.c_int, [C.POINTER(QConvDesc), _P, _P, _P, _P]),
    "miq_qconv2d_nhwc_i8_dequant": (C.c_int, [C.POINTER(QConvDesc), _P, _P, _P, _P, _P, _P]),
    "miq_bmm_i32": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "miq_fprop_nhwc_f32": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, _P]),
    "miq_bprop_nhwc_f32": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, _P]),
    "miq_grad_nhwc_f32": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, _P]),
    "miq_grad_nhwc_f32_workspace_size": (
        C.c_int, [_I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, C.POINTER(C.c_size_t)]),
    "miq_grad_nhwc_f32_noalloc": (C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, _P]),
    "miq_grad_nhwc_f32_ws": (
        C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(Conv2DParams), _I, _P, C.c_size_t, _P]),
    "miq_block_fprop_nhwc_f32": (
        C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _P, _I, _I, _P]),
    "miq_block_bprop_nhwc_f32": (
        C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _I, _P]),
    "miq_block_grad_nhwc_f32": (
        C.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _P, _I, _I, _P]),
    "miq_plan_block_f32": (C.c_int, [_I, _I, _I, _I, _I, _I, _I, _I, C.POINTER(BlockConv2DParams), _I, _PI]),
}

_lib = None


class MiqError(RuntimeError):
    """A non-OK status of the C-ABI; ``status`` holds the miq_status code."""

    def __init__(self, status: int, entry: str, message: str):
        super().__init__(f"{entry}: {message} (status {status})")
        self.status = status


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m my_own_cnn_amd.build` "
                "(the HIP library is required; there is no CPU fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, entry: str) -> None:
    if status != MIQ_OK:
        msg = lib().miq_last_error_message().decode(errors="replace")
        raise MiqError(status, entry, msg)
