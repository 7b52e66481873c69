"""The five int8 convolution workloads of the benchmark and their synthetic inputs.

Inputs are generated with splitmix64 (a counter-based 64-bit generator: number i of stream
`seed` is the splitmix64 finaliser of seed + (i+1) * 0x9E3779B97F4A7C15) and explicit
integer mappings, so numpy, the C test oracle and any other implementation produce the
same bytes.  Stream seeds are 42 ^ (cfg_id << 8) ^ tensor_id with tensor ids x=1, w=2,
bias=3, w_scale=4 (42 is the reference benchmark's default seed, src/main.cpp:39).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
TENSOR_IDS = {"x": 1, "w": 2, "bias": 3, "w_scale": 4}


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs start .. start+count-1 of the stream `seed` (uint64)."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    z = np.uint64(seed) + i * GOLDEN
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def fill_i8_uniform(count: int, seed: int, lo: int, hi: int) -> np.ndarray:
    """lo + floor(hi32(u) * (hi - lo + 1) / 2^32) as int8."""
    u = splitmix64(seed, 0, count)
    v = ((u >> np.uint64(32)) * np.uint64(hi - lo + 1)) >> np.uint64(32)
    return (v.astype(np.int64) + lo).astype(np.int8)


def fill_i8_relu_half(count: int, seed: int) -> np.ndarray:
    """0 when the top bit of u is clear, else 1 + floor(lo32(u) * 127 / 2^32)."""
    u = splitmix64(seed, 0, count)
    v = (((u & np.uint64(0xFFFFFFFF)) * np.uint64(127)) >> np.uint64(32)).astype(np.int64) + 1
    return np.where((u >> np.uint64(63)) != 0, v, 0).astype(np.int8)


def fill_i32_uniform(count: int, seed: int, lo: int, hi: int) -> np.ndarray:
    u = splitmix64(seed, 0, count)
    v = ((u >> np.uint64(32)) * np.uint64(hi - lo + 1)) >> np.uint64(32)
    return (v.astype(np.int64) + lo).astype(np.int32)


def fill_f32_uniform(count: int, seed: int, lo: float, hi: float) -> np.ndarray:
    """lo + f * (hi - lo) in single precision, f = top 24 bits of u / 2^24."""
    u = splitmix64(seed, 0, count)
    f = (u >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    span = np.float32(hi32 - lo32)
    return (lo32 + (f * span).astype(np.float32)).astype(np.float32)


@dataclass(frozen=True)
class Workload:
    cfg_id: int
    name: str
    n: int
    h: int
    w: int
    c: int
    k: int
    r: int
    s: int
    stride: int
    pad: int
    relu: bool
    x_dist: str = "uniform"  # or "relu_half": 0 w.p. 1/2, else uniform[1, 127]
    groups: int = 1
    in_scale: float = 0.02
    out_scale: float = 1.0

    @property
    def ho(self) -> int:
        return (self.h + 2 * self.pad - (self.r - 1) - 1) // self.stride + 1

    @property
    def wo(self) -> int:
        return (self.w + 2 * self.pad - (self.s - 1) - 1) // self.stride + 1

    @property
    def conv7(self):
        """(pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, groups)"""
        return (self.pad, self.pad, self.stride, self.stride, 1, 1, self.groups)

    @property
    def ops(self) -> int:
        """2 * N * Ho * Wo * K * R * S * C / groups (the reference's count, src/main.cpp:143-145)."""
        return 2 * self.n * self.ho * self.wo * self.k * self.r * self.s * (self.c // self.groups)

    @property
    def x_bytes(self) -> int:
        return self.n * self.h * self.w * self.c

    @property
    def w_bytes(self) -> int:
        return self.k * self.r * self.s * (self.c // self.groups)

    @property
    def y_bytes(self) -> int:
        return self.n * self.ho * self.wo * self.k

    @property
    def bytes(self) -> int:
        """Compulsory HBM traffic: x + w + y (int8) + bias (int32[K]) + scales (f32[K])."""
        return self.x_bytes + self.w_bytes + self.y_bytes + 8 * self.k

    def seed(self, tensor: str) -> int:
        return 42 ^ (self.cfg_id << 8) ^ TENSOR_IDS[tensor]

    def inputs(self) -> Dict[str, np.ndarray]:
        """Synthetic x (NHWC int8), w (KRSC int8), bias (int32[K]), w_scale (f32[K])."""
        if self.x_dist == "relu_half":
            x = fill_i8_relu_half(self.x_bytes, self.seed("x"))
        else:
            x = fill_i8_uniform(self.x_bytes, self.seed("x"), -128, 127)
        w = fill_i8_uniform(self.w_bytes, self.seed("w"), -127, 127)
        return {
            "x": x.reshape(self.n, self.h, self.w, self.c),
            "w": w.reshape(self.k, self.r, self.s, self.c // self.groups),
            "bias": fill_i32_uniform(self.k, self.seed("bias"), -1024, 1024),
            "w_scale": fill_f32_uniform(self.k, self.seed("w_scale"), 1e-3, 1e-2),
        }


WORKLOADS = {
    "tiny": Workload(1, "tiny", 1, 32, 32, 16, 32, 3, 3, 1, 1, relu=False),
    "r50_3x3": Workload(2, "r50_3x3", 32, 56, 56, 64, 64, 3, 3, 1, 1, relu=True),
    "r50_1x1": Workload(3, "r50_1x1", 64, 28, 28, 128, 512, 1, 1, 1, 0, relu=False),
    "down_s2": Workload(4, "down_s2", 32, 56, 56, 128, 256, 3, 3, 2, 1, relu=True, x_dist="relu_half"),
    "stem": Workload(5, "stem", 32, 224, 224, 3, 64, 7, 7, 2, 3, relu=True),
}

HEADLINE = "r50_3x3"  # BASELINE.json configs[1], the metric's layer
