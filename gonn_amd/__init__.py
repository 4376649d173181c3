"""gonn_amd -- MI355X (gfx950) attention core for GoNN.

Hand-written HIP kernels (flash forward, dQ/dK/dV backward, split-KV decode)
behind the C ABI of include/gonn_hip.h, plus the host-side mirror of GoNN's
attention seam (gonn_amd.hip for backend/cuda's entry points, gonn_amd.nn for
nn/flashattn_cuda.go and the fused MultiHeadAttention branch).
"""
from . import _lib, hip, nn  # noqa: F401
from ._lib import GonnHipError  # noqa: F401

__all__ = ["hip", "nn", "GonnHipError"]
