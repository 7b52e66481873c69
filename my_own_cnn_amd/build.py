"""Builds libmiq_qconv.so (HIP kernels + C-ABI + C++ drop-in shim) for gfx950, in-tree.

    python -m my_own_cnn_amd.build          # or: python my_own_cnn_amd/build.py

Every HIP/C++ translation unit is compiled with hipcc for gfx950 only, with packed-FP32
instruction selection disabled and floating-point contraction off (the requantization
epilogue is specified as separate IEEE-754 operations).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libmiq_qconv.so"

ARCH = "gfx950"
SOURCES = [
    "qconv_capi.cpp",
    "qconv_direct.hip",
    "qconv_igemm.hip",
    "qconv_stem.hip",
    "qconv_stem_s2d.hip",
    "qconv_band.hip",
    "qconv_stream.hip",
    "qconv_flat.hip",
    "qconv_pipe.hip",
    "qconv_pointwise.hip",
    "qconv_dot4.hip",
    "gemm_i32.hip",
    "conv_f32.hip",
    "grad_noalloc.hip",
    "qconv_qi32.hip",
    "qconv_qi32_band.hip",
    "qconv_qi32_route.hip",
    "conv_quant_host.cpp",
    "verify.cpp",
    "bench.cpp",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmiq_qconv")
    return exe


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-mcode-object-version=5",  # loadable by the HIP runtime PyTorch bundles as well as /opt/rocm's
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in res.stdout.splitlines()
        if "packed-fp32-ops" not in ln and "is not a recognized feature" not in ln
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the shared library; always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    flags = common_flags()

    def compile_one(src: str) -> Path:
        obj = BUILD / (src + ".o")
        cmd = [cc, *flags, "-c", str(CSRC / src), "-o", str(obj)]
        if src.endswith(".cpp"):
            cmd.insert(1, "-xhip")
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    jobs = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
