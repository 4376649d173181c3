"""GPU checks of the HIP backend's fp64 elementwise ops (gonn_hip_unary_f64 /
gonn_hip_binary_f64 and their device-buffer forms): the capability
backend.Elementwiser (backend/backend.go:80-92). Bar: max absolute
difference 1e-12 against host libm, the reference's GPU-vs-CPU bar
(tensor/cuda_dispatch_test.go:48-106, inputs N(0,1), divisor N(0,1)+3).
Known-answer values pin the host-side formulas (a CPU test)."""
import math

import numpy as np
import pytest
from scipy.special import erf

from gonn_amd import _lib, backend, hip
from tests._util import say

torch = pytest.importorskip("torch")

_HOST = {
    _lib.GONN_UN_RELU: lambda x: np.where(x > 0, x, 0.0),
    _lib.GONN_UN_SIGMOID: lambda x: 1.0 / (1.0 + np.exp(-x)),
    _lib.GONN_UN_TANH: np.tanh,
    _lib.GONN_UN_EXP: np.exp,
    _lib.GONN_UN_LOG: np.log,
    _lib.GONN_UN_GELU: lambda x: 0.5 * x * (1.0 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3))),
    _lib.GONN_UN_SILU: lambda x: x / (1.0 + np.exp(-x)),
    _lib.GONN_UN_GELU_EXACT: lambda x: 0.5 * x * (1.0 + erf(x / math.sqrt(2.0))),
}
_BIN = {_lib.GONN_BIN_ADD: np.add, _lib.GONN_BIN_SUB: np.subtract,
        _lib.GONN_BIN_MUL: np.multiply, _lib.GONN_BIN_DIV: np.divide}

# f(x) at points where the value is known independently of the formulas above.
_KNOWN = {
    _lib.GONN_UN_RELU: [(-1.5, 0.0), (2.5, 2.5)],
    _lib.GONN_UN_SIGMOID: [(0.0, 0.5), (math.log(3.0), 0.75)],
    _lib.GONN_UN_TANH: [(0.0, 0.0), (math.log(2.0), 0.6)],          # (4-1)/(4+1)
    _lib.GONN_UN_EXP: [(0.0, 1.0), (1.0, math.e)],
    _lib.GONN_UN_LOG: [(1.0, 0.0), (math.e, 1.0)],
    _lib.GONN_UN_GELU: [(0.0, 0.0)],
    _lib.GONN_UN_SILU: [(0.0, 0.0), (math.log(3.0), 0.75 * math.log(3.0))],
    _lib.GONN_UN_GELU_EXACT: [(0.0, 0.0), (1.0, 0.8413447460685429), (-1.0, -0.15865525393145707)],
}


def _input(kind, n, seed):
    x = np.random.default_rng(seed).standard_normal(n)
    return np.abs(x) + 0.05 if kind == _lib.GONN_UN_LOG else x


def test_host_formulas_known_answers():
    for kind, pts in _KNOWN.items():
        for x, y in pts:
            assert abs(float(_HOST[kind](np.array([x]))[0]) - y) <= 1e-15, (kind, x)
    # The tanh form approximates the erf form to within 1e-3 on [-6, 6].
    xs = np.linspace(-6, 6, 10001)
    assert np.max(np.abs(_HOST[_lib.GONN_UN_GELU](xs) - _HOST[_lib.GONN_UN_GELU_EXACT](xs))) < 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("kind", sorted(_HOST))
@pytest.mark.parametrize("n", [1, 3, 4096, 1000003])
def test_unary_matches_host(kind, n):
    say(f"[unary] kind={kind} n={n}")
    x = _input(kind, n, 11 + kind)
    got = hip.Unary(kind, x)
    err = float(np.max(np.abs(got - _HOST[kind](x))))
    assert err <= 1e-12, err
    pts = _KNOWN[kind]
    kv = hip.Unary(kind, np.array([p[0] for p in pts]))
    assert np.max(np.abs(kv - np.array([p[1] for p in pts]))) <= 1e-15


@pytest.mark.gpu
@pytest.mark.parametrize("kind", sorted(_BIN))
@pytest.mark.parametrize("n", [1, 4096, 1000003])
def test_binary_matches_host(kind, n):
    say(f"[binary] kind={kind} n={n}")
    rng = np.random.default_rng(12 + kind)
    a, b = rng.standard_normal(n), rng.standard_normal(n) + 3.0
    got = hip.Binary(kind, a, b)
    # +, -, * and / are correctly rounded on both sides: bit-identical.
    assert np.array_equal(got, _BIN[kind](a, b))


@pytest.mark.gpu
def test_device_buffers_and_dispatch():
    n = (1 << 20) + 5
    x = torch.randn(n, dtype=torch.float64, device="cuda")
    y = torch.randn(n, dtype=torch.float64, device="cuda") + 3.0
    out = torch.empty_like(x)
    import ctypes
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    bx, by, bo = (_lib.Buf(t.data_ptr(), t.numel() * 8, _lib.GONN_F64) for t in (x, y, out))
    lib = _lib.load()
    _lib.check(lib.gonn_hip_unary_f64_dev(_lib.GONN_UN_TANH, ctypes.byref(bx), ctypes.byref(bo), n, st), "unary dev")
    torch.cuda.synchronize()
    assert (out - torch.tanh(x)).abs().max().item() <= 1e-12
    _lib.check(lib.gonn_hip_binary_f64_dev(_lib.GONN_BIN_DIV, ctypes.byref(bx), ctypes.byref(by),
                                           ctypes.byref(bo), n, st), "binary dev")
    torch.cuda.synchronize()
    assert torch.equal(out, x / y)

    # tensor/dispatch.go path: policy forced to 0 as cuda_dispatch_test.go:23-36 does.
    prev, prevp = backend.Use(backend.HIPBackend()), backend.GetDispatchPolicy()
    backend.SetDispatchPolicy(backend.DispatchPolicy(0, 0))
    try:
        a = np.random.default_rng(3).standard_normal(5000)
        o = np.empty_like(a)
        assert backend.dispatch_unary(backend.UnarySiLU, a, o)
        assert np.max(np.abs(o - _HOST[_lib.GONN_UN_SILU](a))) <= 1e-12
        assert backend.dispatch_binary(backend.BinarySub, a, a[::-1].copy(), o)
        assert np.array_equal(o, a - a[::-1])
        assert not backend.dispatch_unary(backend.UnaryNone, a, o)
    finally:
        backend.Use(prev)
        backend.SetDispatchPolicy(prevp)
