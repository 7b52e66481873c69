"""The allocation-free fp32 grad entry point (miq_grad_nhwc_f32_noalloc) against the ordered
one it mirrors (miq_grad_nhwc_f32, AUTO), through the C-ABI: the same bits on two calls in a
row, the second smaller than the first (the shared device array keeps the first call's
partial sums, which the second must overwrite), and a clear rejection of shapes whose
partial sums exceed the array."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
import my_own_cnn_amd as M
from my_own_cnn_amd import _capi

pytestmark = pytest.mark.gpu

SHAPES = [
    # name, n, h, w, c, k, r, s, conv7: multi-split MFMA GEMM, then a smaller depthwise call
    ("igemm_56x56_n8", 8, 56, 56, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
    ("depthwise_n2", 2, 28, 28, 64, 64, 3, 3, (1, 1, 1, 1, 1, 1, 64)),
    ("igemm_small", 1, 20, 20, 32, 32, 3, 3, (1, 1, 1, 1, 1, 1, 1)),
]


def _call(fn, xd, dyd, dw, shape, conv):
    n, h, w, c, k, r, s = shape
    p = _capi.Conv2DParams(*conv)
    st = fn(C.c_void_p(xd.data_ptr()), C.c_void_p(dyd.data_ptr()), C.c_void_p(dw.data_ptr()), n, h, w, c, r, s, k,
            C.byref(p), 0, None)
    assert st == _capi.MIQ_OK, M.lib().miq_last_error_message()


def test_noalloc_grad_matches_the_ordered_entry_point(device):
    lib = M.lib()
    sizes = []
    for i, (name, n, h, w, c, k, r, s, conv) in enumerate(SHAPES):
        rng = np.random.default_rng(40 + i)
        ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
        x = rng.uniform(-1, 1, size=(n, h, w, c)).astype(np.float32)
        dy = rng.uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)
        xd, dyd = torch.from_numpy(x).to(device), torch.from_numpy(dy).to(device)
        wshape = (k, r, s, c // conv[6])
        sizes.append(M.grad_workspace_size(n, h, w, c, r, s, k, conv))
        ref = torch.full(wshape, 7.0, dtype=torch.float32, device=device)
        got = torch.full(wshape, -3.0, dtype=torch.float32, device=device)
        _call(lib.miq_grad_nhwc_f32, xd, dyd, ref, (n, h, w, c, k, r, s), conv)
        _call(lib.miq_grad_nhwc_f32_noalloc, xd, dyd, got, (n, h, w, c, k, r, s), conv)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref.cpu().numpy().view(np.uint32),
                                      err_msg=name)
        if i == 0:  # the values themselves: integer inputs make every partial sum exact in fp32,
            # so the result must equal cpu_grad_nhwc bit for bit
            xi = rng.integers(-3, 4, size=x.shape).astype(np.float32)
            dyi = rng.integers(-3, 4, size=dy.shape).astype(np.float32)
            want = oracle.grad_f32(xi, dyi, wshape, conv)
            one = torch.empty(wshape, dtype=torch.float32, device=device)
            _call(lib.miq_grad_nhwc_f32_noalloc, torch.from_numpy(xi).to(device), torch.from_numpy(dyi).to(device), one,
                  (n, h, w, c, k, r, s), conv)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(one.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert sizes[0] > sizes[1] > 0, sizes  # second call smaller, both through the shared array


def test_noalloc_grad_rejects_what_does_not_fit(device):
    lib = M.lib()
    conv = (1, 1, 1, 1, 1, 1, 1)
    n, h, w, c, k, r, s = 32, 56, 56, 256, 256, 3, 3
    need = M.grad_workspace_size(n, h, w, c, r, s, k, conv)
    assert need > 32 << 20
    x = torch.empty((n, h, w, c), dtype=torch.float32, device=device)
    dy = torch.empty((n, h, w, k), dtype=torch.float32, device=device)
    dw = torch.empty((k, r, s, c), dtype=torch.float32, device=device)
    p = _capi.Conv2DParams(*conv)
    st = lib.miq_grad_nhwc_f32_noalloc(C.c_void_p(x.data_ptr()), C.c_void_p(dy.data_ptr()),
                                       C.c_void_p(dw.data_ptr()), n, h, w, c, r, s, k, C.byref(p), 0, None)
    assert st == _capi.MIQ_ERR_UNSUPPORTED
    assert b"allocation-free" in lib.miq_last_error_message()


def test_noalloc_grad_in_a_graph(device):
    """miq_grad_nhwc_f32_noalloc recorded into a HIP graph (torch.cuda.graph on a side stream)
    and replayed three times, with eager work and synchronisations between replays: every
    replay gives the ordered entry point's bits, and the captured call allocates nothing (the
    device's free memory does not drop by anything near the 28.9 MB workspace the allocating
    entry point would need)."""
    lib = M.lib()
    name, n, h, w, c, k, r, s, conv = SHAPES[0]
    rng = np.random.default_rng(77)
    ho, wo = oracle.conv_output_shape(n, h, w, c, r, s, k, conv)
    xd = torch.from_numpy(rng.uniform(-1, 1, size=(n, h, w, c)).astype(np.float32)).to(device)
    dyd = torch.from_numpy(rng.uniform(-1, 1, size=(n, ho, wo, k)).astype(np.float32)).to(device)
    wshape = (k, r, s, c // conv[6])
    need = M.grad_workspace_size(n, h, w, c, r, s, k, conv)
    assert need > 16 << 20
    ref = torch.empty(wshape, dtype=torch.float32, device=device)
    _call(lib.miq_grad_nhwc_f32, xd, dyd, ref, (n, h, w, c, k, r, s), conv)
    got = torch.empty(wshape, dtype=torch.float32, device=device)
    _call(lib.miq_grad_nhwc_f32_noalloc, xd, dyd, got, (n, h, w, c, k, r, s), conv)  # first call on the device
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    free0 = torch.cuda.mem_get_info()[0]
    graph = torch.cuda.CUDAGraph()
    p = _capi.Conv2DParams(*conv)
    print("noalloc grad graph: capture", flush=True)
    with torch.cuda.graph(graph, stream=side):
        st = lib.miq_grad_nhwc_f32_noalloc(C.c_void_p(xd.data_ptr()), C.c_void_p(dyd.data_ptr()),
                                           C.c_void_p(got.data_ptr()), n, h, w, c, r, s, k, C.byref(p), 0,
                                           C.c_void_p(side.cuda_stream))
    assert st == _capi.MIQ_OK, lib.miq_last_error_message()
    torch.cuda.synchronize()
    want = ref.cpu().numpy().view(np.uint32)
    for rep in range(3):
        got.fill_(float(rep) - 5.0)
        torch.cuda.synchronize()
        print(f"noalloc grad graph: replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want, err_msg=f"replay {rep}")
    free1 = torch.cuda.mem_get_info()[0]
    assert free0 - free1 < need // 2, (free0, free1, need)
