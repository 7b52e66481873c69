"""MI355X-native quantized NHWC convolution (int8 MFMA implicit GEMM for gfx950).

The compute lives in libmiq_qconv.so (hand-written HIP kernels behind the C-ABI of
include/miq_qconv.h); this package is the Python binding of that ABI and the workload
definitions of the benchmark.  There is no CPU fallback: every entry point raises if the
library has not been built.
"""
from .conv import (BlockConv2DParams, bmm_i32, bmm_matmul_i32, conv2d_nhwc_f32, launch_fprop_nhwc, launch_bprop_nhwc, launch_grad_nhwc, grad_workspace_size,
                   launch_block_fprop_nhwc, launch_block_bprop_nhwc, launch_block_grad_nhwc, plan_block_f32, Conv2DParams, DataType, MiqError, QConvDesc, QParamsS5, QParamsU8,
                   infer_block_conv_shape, infer_conv_shape, launch_block_fprop_nhwc_qi32, launch_fprop_nhwc_qi32,
                   fprop_nhwc_qi32_algo, plan_qi32, plan_block_qi32, qi32_workspace_size,
                   make_desc, plan, plan_f32, qconv2d_nhwc_i8, qconv2d_nhwc_i8_acc32, qconv2d_nhwc_i8_dequant, qparams_array)
from ._capi import LIB_PATH, lib
from .workloads import HEADLINE, WORKLOADS, Workload

__all__ = [
    "bmm_i32", "bmm_matmul_i32", "conv2d_nhwc_f32", "launch_fprop_nhwc", "launch_bprop_nhwc", "launch_grad_nhwc", "grad_workspace_size",
    "launch_block_fprop_nhwc", "launch_block_bprop_nhwc", "launch_block_grad_nhwc", "plan_block_f32", "BlockConv2DParams", "Conv2DParams", "DataType", "MiqError", "QConvDesc", "QParamsS5", "QParamsU8",
    "infer_block_conv_shape", "infer_conv_shape", "launch_block_fprop_nhwc_qi32", "launch_fprop_nhwc_qi32",
    "fprop_nhwc_qi32_algo", "plan_qi32", "plan_block_qi32", "qi32_workspace_size",
    "make_desc", "plan", "plan_f32", "qconv2d_nhwc_i8", "qconv2d_nhwc_i8_acc32", "qconv2d_nhwc_i8_dequant", "qparams_array",
    "LIB_PATH", "lib", "HEADLINE", "WORKLOADS", "Workload",
]
