"""GPU checks of the HIP backend's fp64 GEMM (gonn_hip_gemm_f64 /
gonn_hip_gemm_f64_dev: rocBLAS on gfx950, and a kernel of its own for the
skinny C = A W^T shapes of a decoding step) and of the MHA running its
projections through it. Bar: max absolute difference 1e-10, the
reference's GPU-vs-CPU GEMM bar (tensor/cuda_dispatch_test.go:127-131); the
CPU side is numpy's fp64 matmul (an independent BLAS), and the small cases
are also checked against a naive loop (tests/test_backend.py)."""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _ref(A, B, batch, m, k, n, ta, tb):
    A = A.reshape(batch, *((k, m) if ta else (m, k)))
    B = B.reshape(batch, *((n, k) if tb else (k, n)))
    return np.matmul(A.transpose(0, 2, 1) if ta else A, B.transpose(0, 2, 1) if tb else B).reshape(-1)


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (3, 7, 33, 5), (2, 129, 64, 257), (1, 1024, 1024, 1024)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_device_gemm_matches_numpy(shape, ta, tb):
    from gonn_amd import hip
    batch, m, k, n = shape
    say(f"[gemm] {shape} ta={ta} tb={tb}")
    rng = np.random.default_rng(sum(shape) + 2 * ta + tb)
    A = rng.standard_normal(batch * m * k)
    B = rng.standard_normal(batch * k * n)
    got = hip.Gemm(A, B, batch, m, k, n, ta, tb)
    ref = _ref(A, B, batch, m, k, n, ta, tb)
    err = float(np.max(np.abs(got - ref)))
    say(f"[gemm] max abs err {err:.2e}")
    assert err <= 1e-10


@pytest.mark.parametrize("shape", [(1, 128, 16), (7, 256, 33), (16, 128, 1), (33, 384, 100),
                                   (64, 4096, 4096), (64, 4096, 12288), (48, 512, 4100),
                                   (65, 128, 48), (100, 256, 200), (256, 4096, 4096),
                                   (128, 4096, 12288), (200, 384, 136), (200, 256, 4100),
                                   (130, 128, 8200)],
                         ids=lambda s: "x".join(map(str, s)))
def test_skinny_gemm_path(shape, monkeypatch):
    """The skinny kernel (C = A W^T, m <= 256, k % 128 == 0: the decoding
    step's projections; row chunks of 64, 16 and 32 columns per workgroup,
    column tile counts with and without the XCD grouping) against numpy at the backend's bar, on host and
    device buffers, and against the rocBLAS path of the same call
    (GONN_HIP_GEMM=rocblas)."""
    from gonn_amd import _lib, hip
    import ctypes
    m, k, n = shape
    say(f"[gemm skinny] m={m} k={k} n={n}")
    rng = np.random.default_rng(m + k + n)
    A = rng.standard_normal(m * k)
    W = rng.standard_normal(n * k)
    ref = _ref(A, W, 1, m, k, n, False, True)
    got = hip.Gemm(A, W, 1, m, k, n, False, True)
    err = float(np.max(np.abs(got - ref)))
    say(f"[gemm skinny] host max abs err {err:.2e}")
    assert err <= 1e-10
    dA, dW = (torch.from_numpy(x).cuda() for x in (A, W))
    out = {}
    for path in ("skinny", "rocblas"):
        if path == "rocblas":
            monkeypatch.setenv("GONN_HIP_GEMM", "rocblas")
        else:
            monkeypatch.delenv("GONN_HIP_GEMM", raising=False)
        C = torch.full((m * n,), float("nan"), dtype=torch.float64, device="cuda")
        bufs = [_lib.Buf(t.data_ptr(), t.numel() * 8, _lib.GONN_F64) for t in (dA, dW, C)]
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(_lib.load().gonn_hip_gemm_f64_dev(ctypes.byref(bufs[0]), ctypes.byref(bufs[1]),
                                                     ctypes.byref(bufs[2]), 1, m, k, n, 0, 1, st),
                   "gemm_f64_dev")
        torch.cuda.synchronize()
        out[path] = C.cpu().numpy()
        assert np.all(np.isfinite(out[path])), path
        assert float(np.max(np.abs(out[path] - ref))) <= 1e-10, path
    # two fp64 summation orders: equal to rounding
    assert float(np.max(np.abs(out["skinny"] - out["rocblas"]))) <= 1e-11


def test_device_gemm_dev_buffers():
    from gonn_amd import _lib, hip
    import ctypes
    batch, m, k, n = 4, 96, 80, 112
    A = torch.randn(batch, k, m, dtype=torch.float64, device="cuda")  # stored (k, m): transA
    B = torch.randn(batch, k, n, dtype=torch.float64, device="cuda")
    C = torch.empty(batch, m, n, dtype=torch.float64, device="cuda")
    bufs = [_lib.Buf(t.data_ptr(), t.numel() * 8, _lib.GONN_F64) for t in (A, B, C)]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().gonn_hip_gemm_f64_dev(ctypes.byref(bufs[0]), ctypes.byref(bufs[1]),
                                                 ctypes.byref(bufs[2]), batch, m, k, n, 1, 0, st),
               "gemm_f64_dev")
    ref = torch.matmul(A.transpose(1, 2), B)
    torch.cuda.synchronize()
    assert (C - ref).abs().max().item() <= 1e-10


def test_mha_with_hip_backend_projections():
    from gonn_amd import backend, nn
    E, H, B, T = 256, 4, 2, 64
    s = 1.0 / math.sqrt(E)
    p = {}
    for i, nme in enumerate(("q", "k", "v", "o")):
        p["W" + nme] = randn((E, E), 900 + 2 * i).astype(np.float64) * s
        p["b" + nme] = randn((E,), 901 + 2 * i).astype(np.float64) * 0.1
    x = randn((B, T, E), 910).astype(np.float64)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    ref = oracle.mha_fwd(x, x, x, p, H, causal=True)
    cpu = mha.forward_fused(x, x, x, True)
    prev = backend.Use(backend.HIPBackend())
    try:
        dev = mha.forward_fused(x, x, x, True)
    finally:
        backend.Use(prev)
    assert_close(dev, ref, "fp32", "MHA, projections on the HIP backend")
    assert np.max(np.abs(dev - cpu)) <= 1e-9


def test_device_gemm_dev_empty_inner_dim_zeroes_output():
    from gonn_amd import _lib
    import ctypes
    A = torch.empty(0, dtype=torch.float64, device="cuda")
    C = torch.full((3, 5, 7), 9.0, dtype=torch.float64, device="cuda")
    bufs = [_lib.Buf(A.data_ptr(), 0, _lib.GONN_F64), _lib.Buf(A.data_ptr(), 0, _lib.GONN_F64),
            _lib.Buf(C.data_ptr(), C.numel() * 8, _lib.GONN_F64)]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().gonn_hip_gemm_f64_dev(ctypes.byref(bufs[0]), ctypes.byref(bufs[1]),
                                                 ctypes.byref(bufs[2]), 3, 5, 0, 7, 0, 0, st),
               "gemm_f64_dev k=0")
    torch.cuda.synchronize()
    assert C.abs().max().item() == 0.0
