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
"""
from __future__ import annotations

import threading

import numpy as np

from . import hip


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
