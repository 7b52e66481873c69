"""Loaders of the committed golden fixtures (inputs regenerated where the fixture stores
only outputs).  Shared by the CPU and GPU tests."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from tests.golden.make_golden import (FILTER_ZP, INT8_SHAPES, input_zero_points, int8_case_inputs,
                                      quant_codes)

HERE = Path(__file__).resolve().parent


def quant_conv_test_cases():
    """name -> dict(kind, x, w, conv, zp, fzp, block, y) of the reference's four cases."""
    exp = np.load(HERE / "quant_conv_test.npz")
    out = {}
    for kind in ("u8", "s5"):
        out[f"regular_{kind}"] = dict(
            kind=kind, x=quant_codes(kind, 240, 1).reshape(2, 5, 6, 4), w=quant_codes(kind, 72, 7).reshape(6, 3, 2, 2),
            conv=(1, 0, 1, 1, 1, 1, 2), zp=input_zero_points(kind, 2), fzp=FILTER_ZP[kind], block=(0, 0),
            y=exp[f"regular_{kind}"])
        out[f"blocked_{kind}"] = dict(
            kind=kind, x=quant_codes(kind, 288, 3).reshape(2, 6, 6, 4),
            w=quant_codes(kind, 1080, 9).reshape(5, 2, 3, 3, 3, 4), conv=(1, 1, 1, 1, 1, 1, 1),
            zp=input_zero_points(kind, 2), fzp=FILTER_ZP[kind], block=(2, 3), y=exp[f"blocked_{kind}"])
    return out


def qi32_cases():
    z = np.load(HERE / "qi32_cases.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    out = {}
    for nm in names:
        d = {k.split("/")[1]: z[k] for k in z.files if k.split("/")[0] == nm}
        out[nm] = dict(kind=str(d["kind"]), x=d["x"], w=d["w"], conv=tuple(int(v) for v in d["conv"]),
                       zp=d["zp"], fzp=int(d["fzp"]), block=tuple(int(v) for v in d["block"]), y=d["y"])
    return out


def int8_cases():
    z = np.load(HERE / "int8_cases.npz")
    out = {}
    for idx, (name, xshape, wshape3, conv) in enumerate(INT8_SHAPES):
        k, r, s = wshape3
        wshape = (k, r, s, xshape[3] // conv[6])
        x, w = int8_case_inputs(idx, name, xshape, wshape)
        out[name] = dict(x=x, w=w, conv=tuple(conv), y=z[f"{name}/y"])
    return out


def config_goldens():
    with open(HERE / "configs.json") as f:
        return json.load(f)


def c1_acc():
    return np.load(HERE / "c1_tiny.npz")["acc"]


# Full-size float-code problems (the reference's launch_fprop_nhwc_qi32 API at the C2 and C4
# shapes): inputs regenerated from splitmix64 streams, outputs pinned by sha256 in
# qi32_full.json (written by make_qi32_full.py from the reference's cpu_fprop_nhwc_qi32).
QI32_FULL = {
    # name: (kind, workload, code range, seed)
    "c2_u8": ("u8", "r50_3x3", (0.0, 255.0), 7100),
    "c2_s5": ("s5", "r50_3x3", (-16.0, 15.0), 7200),
    "c4_u8": ("u8", "down_s2", (0.0, 255.0), 7300),
    "c5_u8": ("u8", "stem", (0.0, 255.0), 7400),
}


def qi32_full_inputs(name: str):
    """(kind, x, w, conv7, in_zp, f_zp) of a full-size float-code problem: fractional codes
    uniform over the kind's code range, per-image input zero points, one filter zero point."""
    from my_own_cnn_amd.workloads import WORKLOADS, fill_f32_uniform, fill_i32_uniform

    kind, wl_name, (lo, hi), seed = QI32_FULL[name]
    wl = WORKLOADS[wl_name]
    x = fill_f32_uniform(wl.n * wl.h * wl.w * wl.c, seed, lo, hi).reshape(wl.n, wl.h, wl.w, wl.c)
    w = fill_f32_uniform(wl.k * wl.r * wl.s * wl.c, seed + 1, lo, hi).reshape(wl.k, wl.r, wl.s, wl.c)
    zlo, zhi = (0, 255) if kind == "u8" else (-128, 127)
    zp = fill_i32_uniform(wl.n, seed + 2, zlo, zhi)
    fzp = int(fill_i32_uniform(1, seed + 3, zlo, zhi)[0])
    conv = (wl.pad, wl.pad, wl.stride, wl.stride, 1, 1, wl.groups)
    return kind, x, w, conv, zp, fzp


def qi32_full_goldens():
    with open(HERE / "qi32_full.json") as f:
        return json.load(f)
