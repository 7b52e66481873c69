"""The CPU oracle against the golden vectors written by the reference's own cpu_ref.cpp."""
import hashlib

import numpy as np
import pytest

import oracle
from my_own_cnn_amd import workloads as W
from tests.golden import cases


def test_splitmix64_published_vectors():
    # first outputs of splitmix64 for seeds 0 and 1234567 (Vigna's reference implementation)
    assert [oracle.splitmix64(0, i) for i in range(4)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert [oracle.splitmix64(1234567, i) for i in range(3)] == [
        0x599ED017FB08FC85, 0x2C73F08458540FA5, 0x883EBCE5A3F27C77]


@pytest.mark.parametrize("seed", [0, 1, 42 ^ (2 << 8) ^ 1, 0xFFFFFFFFFFFF])
def test_numpy_generator_matches_c(seed):
    np.testing.assert_array_equal(W.splitmix64(seed, 0, 64), [oracle.splitmix64(seed, i) for i in range(64)])
    np.testing.assert_array_equal(W.fill_i8_uniform(5000, seed, -128, 127), oracle.fill_i8_uniform(5000, seed, -128, 127))
    np.testing.assert_array_equal(W.fill_i8_uniform(5000, seed, -127, 127), oracle.fill_i8_uniform(5000, seed, -127, 127))
    np.testing.assert_array_equal(W.fill_i8_relu_half(5000, seed), oracle.fill_i8_relu_half(5000, seed))
    np.testing.assert_array_equal(W.fill_i32_uniform(5000, seed, -1024, 1024),
                                  oracle.fill_i32_uniform(5000, seed, -1024, 1024))
    a = W.fill_f32_uniform(5000, seed, 1e-3, 1e-2)
    b = oracle.fill_f32_uniform(5000, seed, 1e-3, 1e-2)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_generator_ranges():
    x = W.fill_i8_uniform(200000, 7, -128, 127)
    assert x.min() == -128 and x.max() == 127
    w = W.fill_i8_uniform(200000, 8, -127, 127)
    assert w.min() == -127 and w.max() == 127
    r = W.fill_i8_relu_half(200000, 9)
    assert r.min() == 0 and r.max() == 127 and abs((r == 0).mean() - 0.5) < 0.01
    b = W.fill_i32_uniform(200000, 10, -1024, 1024)
    assert b.min() == -1024 and b.max() == 1024
    s = W.fill_f32_uniform(200000, 11, 1e-3, 1e-2)
    assert s.min() >= np.float32(1e-3) and s.max() < np.float32(1e-2)


@pytest.mark.parametrize("name", ["regular_u8", "regular_s5", "blocked_u8", "blocked_s5"])
def test_quant_conv_test_cases(name):
    c = cases.quant_conv_test_cases()[name]
    y = oracle.conv_qi32(c["x"], c["w"], c["conv"], c["zp"], c["fzp"], c["block"])
    np.testing.assert_array_equal(y, c["y"])


def test_qi32_cases():
    for name, c in cases.qi32_cases().items():
        y = oracle.conv_qi32(c["x"], c["w"], c["conv"], c["zp"], c["fzp"], c["block"])
        np.testing.assert_array_equal(y, c["y"], err_msg=name)


def test_int8_cases():
    for name, c in cases.int8_cases().items():
        y = oracle.conv_i8_acc(c["x"], c["w"], c["conv"])
        np.testing.assert_array_equal(y, c["y"], err_msg=name)


def test_c1_in_full():
    wl = W.WORKLOADS["tiny"]
    inp = wl.inputs()
    np.testing.assert_array_equal(oracle.conv_i8_acc(inp["x"], inp["w"], wl.conv7), cases.c1_acc())


@pytest.mark.parametrize("name", list(W.WORKLOADS))
def test_config_accumulators(name):
    wl = W.WORKLOADS[name]
    g = cases.config_goldens()[name]
    inp = wl.inputs()
    assert hashlib.sha256(inp["x"].tobytes()).hexdigest() == g["x_sha256"]
    assert hashlib.sha256(inp["w"].tobytes()).hexdigest() == g["w_sha256"]
    acc = oracle.conv_i8_acc(inp["x"], inp["w"], wl.conv7)
    assert list(acc.shape) == g["shape"]
    flat = acc.reshape(-1)
    np.testing.assert_array_equal(flat[::g["sample_stride"]], g["samples"])
    assert hashlib.sha256(acc.tobytes()).hexdigest() == g["acc_sha256"]


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref (the reference's cpu_ref.cpp) not built here")
def test_oracle_against_reference_random():
    rng = np.random.default_rng(7)
    for trial in range(60):
        groups = int(rng.choice([1, 2, 3]))
        cg = int(rng.integers(1, 5))
        kg = int(rng.integers(1, 4))
        n, h, w = int(rng.integers(1, 3)), int(rng.integers(1, 9)), int(rng.integers(1, 9))
        r, s = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        conv = (int(rng.integers(0, 3)), int(rng.integers(0, 3)), int(rng.integers(1, 3)), int(rng.integers(1, 3)),
                int(rng.integers(1, 3)), int(rng.integers(1, 3)), groups)
        c, k = cg * groups, kg * groups
        if oracle.conv_output_shape(n, h, w, c, r, s, k, conv) is None:
            continue
        kind = "u8" if trial % 2 else "s5"
        lo, hi = (0, 256) if kind == "u8" else (-16, 16)
        x = (rng.integers(lo * 4, hi * 4, size=(n, h, w, c)) / 4.0).astype(np.float32)
        blocked = trial % 3 == 0
        ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
        block = (0, 0)
        if blocked:
            by = int(rng.choice([d for d in range(1, ho + 1) if ho % d == 0]))
            bx = int(rng.choice([d for d in range(1, wo + 1) if wo % d == 0]))
            block = (by, bx)
            wt = rng.integers(lo, hi, size=(k, by, bx, r, s, cg)).astype(np.float32)
        else:
            wt = rng.integers(lo, hi, size=(k, r, s, cg)).astype(np.float32)
        zp = rng.integers(lo, hi, size=n).astype(np.int32)
        fzp = int(rng.integers(lo, hi))
        want, _ = oracle.ref_conv_qi32(kind, x, wt, conv, zp, fzp, block)
        got = oracle.conv_qi32(x, wt, conv, zp, fzp, block)
        np.testing.assert_array_equal(got, want, err_msg=f"trial {trial}")


@pytest.mark.parametrize("name", list(cases.QI32_FULL))
def test_qi32_full_size_against_reference_sha(name):
    """The oracle's float-code convolution at the full C2 / C4 / C5 sizes equals the reference's own
    cpu_fprop_nhwc_qi32 on the same inputs (sha256 of the int32 outputs, written from
    oracle/_ref by tests/golden/make_qi32_full.py)."""
    g = cases.qi32_full_goldens()[name]
    kind, x, w, conv, zp, fzp = cases.qi32_full_inputs(name)
    y = oracle.conv_qi32(x, w, conv, zp, fzp)
    assert list(y.shape) == g["shape"]
    assert hashlib.sha256(y.tobytes()).hexdigest() == g["sha256"]
