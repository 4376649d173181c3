"""gonn_amd.backend -- the compute-target contract around the attention core,
mirroring backend/backend.go:61-78 (Backend: Name, Gemm, Synchronize) and its
process-wide current backend (backend.go:98-118: Use, Current, NewCPU).

Two implementations:
  CPUBackend  row-major fp64 GEMM in numpy (the reference's gonum path,
              backend/cpu.go:20-48, pinned to a naive loop in its tests);
  HIPBackend  the device GEMM of libgonn_hip.so (gonn_hip_gemm_f64, rocBLAS
              fp64 on gfx950), the counterpart of backend/cuda (cuda.go:42-67).
nn.Linear (the MHA projections, nn/linear.go:40-59) multiplies through the
current backend, as tensor.MatMul does through dispatchGemm
(tensor/dispatch.go:111-113).

The optional Elementwiser capability (backend.go:80-92: Unary, Binary on the
UnaryKind / BinaryKind values of backend.go:26-58) is implemented by
HIPBackend only; the CPU backend deliberately lacks it, as in the reference
(backend_test.go:117-126). dispatch_unary / dispatch_binary and the
DispatchPolicy thresholds restate tensor/dispatch.go:44-109.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass

import numpy as np

from . import hip

UnaryNone = -1
(UnaryReLU, UnarySigmoid, UnaryTanh, UnaryExp, UnaryLog, UnaryGELU, UnarySiLU,
 UnaryGELUExact) = range(8)
BinaryAdd, BinarySub, BinaryMul, BinaryDiv = range(4)


class CPUBackend:
    def Name(self) -> str:
        return "cpu"

    def Gemm(self, a, b, batch: int, m: int, k: int, n: int, transA: bool = False,
             transB: bool = False) -> np.ndarray:
        A = np.asarray(a, dtype=np.float64).reshape(batch, *((k, m) if transA else (m, k)))
        B = np.asarray(b, dtype=np.float64).reshape(batch, *((n, k) if transB else (k, n)))
        if transA:
            A = A.transpose(0, 2, 1)
        if transB:
            B = B.transpose(0, 2, 1)
        return np.matmul(A, B).reshape(-1)

    def Synchronize(self) -> None:
        pass


class HIPBackend:
    """Fails loudly without the library or a gfx950 device (no CPU fallback)."""

    def __init__(self):
        if not hip.Available():
            raise RuntimeError("backend: HIP backend needs libgonn_hip.so and a gfx950 device")

    def Name(self) -> str:
        return "hip"

    def Gemm(self, a, b, batch: int, m: int, k: int, n: int, transA: bool = False,
             transB: bool = False) -> np.ndarray:
        return hip.Gemm(a, b, batch, m, k, n, transA, transB)

    def Synchronize(self) -> None:
        pass  # every call of the host GEMM is synchronous

    # Elementwiser. The reference declines (returns False) on any device
    # error so the caller runs its CPU loop (cuda.go:70-106). Here only a kind
    # without a kernel is declined; a device error raises, so a failing device
    # never hides behind a host loop.
    def Unary(self, kind: int, a, out) -> bool:
        if not (0 <= kind <= UnaryGELUExact):
            return False
        hip.Unary(kind, a, out)
        return True

    def Binary(self, kind: int, a, b, out) -> bool:
        if not (0 <= kind <= BinaryDiv):
            return False
        hip.Binary(kind, a, b, out)
        return True


_lock = threading.Lock()
_current = CPUBackend()


def NewCPU() -> CPUBackend:
    return CPUBackend()


def Use(b):
    """Install b as the process-wide backend and return the previous one
    (backend.go Use)."""
    global _current
    if b is None:
        raise ValueError("backend: Use(None)")
    with _lock:
        prev, _current = _current, b
    return prev


def Current():
    return _current


@dataclass(frozen=True)
class DispatchPolicy:
    """Minimum sizes for offloading elementwise ops (tensor/dispatch.go:44-58):
    binary ops never dispatch by default (their host copies cost more than the
    op)."""
    UnaryMinElems: int = 1 << 16
    BinaryMinElems: int = 2 ** 63 - 1


_policy = DispatchPolicy()


def SetDispatchPolicy(p: DispatchPolicy) -> None:
    global _policy
    _policy = p


def GetDispatchPolicy() -> DispatchPolicy:
    return _policy


def dispatch_unary(kind: int, a, out) -> bool:
    """tensor/dispatch.go:74-84: run out = f(a) on the current backend when the
    op has a kernel, a is large enough and the backend has the capability;
    False means the caller runs its own loop."""
    if kind == UnaryNone or np.size(a) < _policy.UnaryMinElems:
        return False
    fn = getattr(Current(), "Unary", None)
    return fn is not None and fn(kind, a, out)


def dispatch_binary(kind: int, a, b, out) -> bool:
    """tensor/dispatch.go:100-109."""
    if np.size(a) < _policy.BinaryMinElems:
        return False
    fn = getattr(Current(), "Binary", None)
    return fn is not None and fn(kind, a, b, out)
