"""gonn_amd.hip -- host side of the HIP attention backend.

Two layers, both over the C ABI (include/gonn_hip.h):

1. The reference's backend/cuda attention entry points under their own names
   and meaning (backend/cuda/cuda.go:125-194), on host fp64 arrays:
       FlashAttnF64(Q, K, V, O, BH, S, d, scale, causal)            cuda.go:128-140
       FlashAttnF64Fwd(Q, K, V, BH, S, d, scale, causal) -> (O, L)  cuda.go:144-160
       FlashAttnF64Bwd(Q, K, V, O, L, dO, BH, S, d, scale, causal)  cuda.go:162-184
       BenchFlashAttnF64(BH, S, d, iters, causal) -> ms             cuda.go:188-194
   The reference returns nothing and ignores device errors; these raise
   GonnHipError on any non-zero status.

2. The device-resident API on torch device tensors (torch only supplies
   device memory and the current HIP stream):
       attn_fwd, attn_bwd, attn_decode

3. KVCache: a device KV cache handle for incremental decoding (new; the
   reference has none), with host fp64 and device-tensor methods.
"""
from __future__ import annotations

import ctypes
import math
import threading

import numpy as np

from . import _lib
from ._lib import (GONN_ATTN_BF16_MFMA, GONN_ATTN_FP32_MFMA, GONN_ATTN_FP64, GONN_BF16,
                   GONN_F32, GONN_I32,
                   GONN_OP_BWD, GONN_OP_DECODE, GONN_OP_FWD, Buf, BwdArgs, DecodeArgs, FwdArgs,
                   GonnHipError, check)

MODES = {"fp32": GONN_ATTN_FP32_MFMA, "bf16": GONN_ATTN_BF16_MFMA,
         GONN_ATTN_FP32_MFMA: GONN_ATTN_FP32_MFMA, GONN_ATTN_BF16_MFMA: GONN_ATTN_BF16_MFMA}
# Modes of the f64 entry points: the two MFMA modes, or "f64" (fp64
# throughout, the precision of the reference's fp64 CUDA seam).
SHIM_MODES = {**MODES, "f64": GONN_ATTN_FP64, GONN_ATTN_FP64: GONN_ATTN_FP64}
_SHIM_MODE_NAMES = {GONN_ATTN_FP32_MFMA: "fp32", GONN_ATTN_BF16_MFMA: "bf16",
                    GONN_ATTN_FP64: "f64"}

_dp = ctypes.POINTER(ctypes.c_double)


# ---------------------------------------------------------------------------
# library queries
# ---------------------------------------------------------------------------
def Available() -> bool:
    """fusedAttnAvailable (nn/flashattn_cuda.go:13) as a runtime query."""
    return bool(_lib.load().gonn_hip_available())


def Supports(D: int, Sq: int, Sk: int) -> bool:
    """Replaces the D == 64 && Tq == Tk gate of nn/attention.go:129."""
    return bool(_lib.load().gonn_hip_attn_supports(int(D), int(Sq), int(Sk)))


def SetAttnMode(mode) -> None:
    """Mode of the f64 entry points: "fp32", "bf16" or "f64"."""
    check(_lib.load().gonn_hip_set_attn_mode(SHIM_MODES[mode]), "SetAttnMode")


def AttnMode() -> str:
    return _SHIM_MODE_NAMES[_lib.load().gonn_hip_get_attn_mode()]


def Version() -> str:
    return _lib.load().gonn_hip_version().decode()


def SelftestMFMA() -> int:
    return int(_lib.load().gonn_hip_selftest_mfma())


def profile_enable(on: bool) -> None:
    check(_lib.load().gonn_hip_profile_enable(int(bool(on))), "profile_enable")


def profile_reset() -> None:
    check(_lib.load().gonn_hip_profile_reset(), "profile_reset")


def profile_read(kernel: str):
    """(total_ms, count) of one kernel stage recorded while profiling was on."""
    tot = ctypes.c_double(0.0)
    n = ctypes.c_int(0)
    check(_lib.load().gonn_hip_profile_read(kernel.encode(), ctypes.byref(tot), ctypes.byref(n)),
          "profile_read")
    return tot.value, n.value


def calib_mfma(random: bool = False):
    """(TFLOP/s, shader GHz) of a fixed bf16 MFMA loop over the whole device,
    on constant operands or (random) distinct uniform values per lane."""
    t, g = ctypes.c_double(0.0), ctypes.c_double(0.0)
    check(_lib.load().gonn_hip_calib_mfma(int(bool(random)), ctypes.byref(t), ctypes.byref(g)),
          "calib_mfma")
    return t.value, g.value


def calib_clock_start(ms: float, stream=None) -> None:
    """Enqueue the shader-clock probe (about `ms` milliseconds) on `stream`."""
    check(_lib.load().gonn_hip_calib_clock_start(float(ms), _stream(stream)), "calib_clock")


def calib_clock_read() -> float:
    """Shader clock (GHz) the last probe saw; after its stream has finished."""
    g = ctypes.c_double(0.0)
    check(_lib.load().gonn_hip_calib_clock_read(ctypes.byref(g)), "calib_clock_read")
    return g.value


# ---------------------------------------------------------------------------
# reference-named f64 entry points
# ---------------------------------------------------------------------------
def _f64(a, n, name):
    a = np.ascontiguousarray(a, dtype=np.float64)
    if a.size != n:
        raise ValueError(f"{name}: expected {n} elements, got {a.size}")
    return a


def _p(a):
    return a.ctypes.data_as(_dp)


def FlashAttnF64(Q, K, V, O, BH: int, S: int, d: int, scale: float, causal: bool) -> None:
    """Fused forward on host fp64 (BH,S,d) arrays; writes O in place."""
    n = BH * S * d
    Q, K, V = (_f64(x, n, "FlashAttnF64") for x in (Q, K, V))
    if not (isinstance(O, np.ndarray) and O.dtype == np.float64 and O.flags.c_contiguous
            and O.size == n):
        raise ValueError("FlashAttnF64: O must be a contiguous float64 array of BH*S*d")
    check(_lib.load().gonn_hip_flash_attn_f64(_p(Q), _p(K), _p(V), _p(O), BH, S, d,
                                              float(scale), int(bool(causal))), "FlashAttnF64")


def FlashAttnF64Fwd(Q, K, V, BH: int, S: int, d: int, scale: float, causal: bool):
    """Training forward: returns (O, L) with L the per-row logsumexp (BH*S)."""
    n = BH * S * d
    Q, K, V = (_f64(x, n, "FlashAttnF64Fwd") for x in (Q, K, V))
    O = np.zeros(n)
    L = np.zeros(BH * S)
    check(_lib.load().gonn_hip_flash_attn_f64_fwd(_p(Q), _p(K), _p(V), _p(O), _p(L), BH, S, d,
                                                  float(scale), int(bool(causal))),
          "FlashAttnF64Fwd")
    return O, L


def FlashAttnF64Bwd(Q, K, V, O, L, dO, BH: int, S: int, d: int, scale: float, causal: bool):
    """Backward from the saved forward tensors: returns (dQ, dK, dV)."""
    n = BH * S * d
    Q, K, V, O, dO = (_f64(x, n, "FlashAttnF64Bwd") for x in (Q, K, V, O, dO))
    L = _f64(L, BH * S, "FlashAttnF64Bwd")
    dQ, dK, dV = np.zeros(n), np.zeros(n), np.zeros(n)
    check(_lib.load().gonn_hip_flash_attn_f64_bwd(_p(Q), _p(K), _p(V), _p(O), _p(L), _p(dO),
                                                  _p(dQ), _p(dK), _p(dV), BH, S, d,
                                                  float(scale), int(bool(causal))),
          "FlashAttnF64Bwd")
    return dQ, dK, dV


def _host_mask(attn_mask, B, H, Sq, Sk):
    if attn_mask is None:
        return None, 0, 0
    m = np.ascontiguousarray(attn_mask, dtype=np.float64)
    sb, sh = mask_strides(m.shape, B, H, Sq, Sk)
    return m, sb, sh


def FlashAttnF64BwdEx(Q, K, V, O, L, dO, B: int, H: int, S: int, d: int, scale: float,
                      causal: bool, kv_len=None, attn_mask=None, Sk=None):
    """General backward on host fp64 arrays (new): Q, O, dO (B*H,S,d), K, V
    (B*H,Sk,d) with Sk = S unless given (cross-attention), the forward's
    optional key padding kv_len[B] and additive attn_mask; returns
    (dQ, dK, dV). O and L come from FlashAttnF64Ex(..., lse=True) with the
    same options."""
    Sk = S if Sk is None else int(Sk)
    n, nk = B * H * S * d, B * H * Sk * d
    Q, O, dO = (_f64(x, n, "FlashAttnF64BwdEx") for x in (Q, O, dO))
    K, V = (_f64(x, nk, "FlashAttnF64BwdEx K/V") for x in (K, V))
    L = _f64(L, B * H * S, "FlashAttnF64BwdEx L")
    kl = None
    if kv_len is not None:
        kl = np.ascontiguousarray(kv_len, dtype=np.int32)
        if kl.shape != (B,):
            raise ValueError(f"FlashAttnF64BwdEx: kv_len must have {B} entries")
    dQ, dK, dV = np.zeros(n), np.zeros(nk), np.zeros(nk)
    m, sb, sh = _host_mask(attn_mask, B, H, S, Sk)
    check(_lib.load().gonn_hip_flash_attn_f64_bwd_masked(
        _p(Q), _p(K), _p(V), _p(O), _p(L), _p(dO), _p(dQ), _p(dK), _p(dV), B, H, S, Sk, d,
        float(scale), int(bool(causal)),
        kl.ctypes.data_as(ctypes.POINTER(ctypes.c_int)) if kl is not None else None,
        _p(m) if m is not None else None, sb, sh), "FlashAttnF64BwdEx")
    return dQ, dK, dV


def FlashAttnF64Ex(Q, K, V, B: int, H: int, Sq: int, Sk: int, d: int, scale: float,
                   causal: bool, kv_len=None, lse: bool = False, attn_mask=None):
    """General fused forward on host fp64 arrays (new; the reference seam is
    Tq == Tk only): Q (B*H,Sq,d), K/V (B*H,Sk,d), optional prefix key padding
    kv_len[B] (keys t >= kv_len[b] masked, ForwardMasked semantics) and
    additive mask attn_mask (WithAttnMask, one of mask_strides' shapes), in the
    current mode. Returns O, or (O, L) when lse is set."""
    Q = _f64(Q, B * H * Sq * d, "FlashAttnF64Ex Q")
    K = _f64(K, B * H * Sk * d, "FlashAttnF64Ex K")
    V = _f64(V, B * H * Sk * d, "FlashAttnF64Ex V")
    O = np.zeros(B * H * Sq * d)
    L = np.zeros(B * H * Sq) if lse else None
    kl = None
    if kv_len is not None:
        kl = np.ascontiguousarray(kv_len, dtype=np.int32)
        if kl.shape != (B,):
            raise ValueError(f"FlashAttnF64Ex: kv_len must have {B} entries")
    m, sb, sh = _host_mask(attn_mask, B, H, Sq, Sk)
    check(_lib.load().gonn_hip_flash_attn_f64_masked(
        _p(Q), _p(K), _p(V), _p(O), _p(L) if L is not None else None, B, H, Sq, Sk, d,
        float(scale), int(bool(causal)),
        kl.ctypes.data_as(ctypes.POINTER(ctypes.c_int)) if kl is not None else None,
        _p(m) if m is not None else None, sb, sh), "FlashAttnF64Ex")
    return (O, L) if lse else O


def Gemm(a, b, batch: int, m: int, k: int, n: int, transA: bool = False,
         transB: bool = False) -> np.ndarray:
    """backend.Backend.Gemm (backend/backend.go:61-78) on the device: row-major
    batched C = op(A) op(B) of host float64 data (A: batch*m*k, B: batch*k*n
    elements); returns the batch*m*n result (flat), like cuda.go:42-67."""
    a = _f64(a, batch * m * k, "Gemm A")
    b = _f64(b, batch * k * n, "Gemm B")
    out = np.zeros(batch * m * n)
    if out.size == 0:
        return out
    check(_lib.load().gonn_hip_gemm_f64(_p(a) if a.size else None, _p(b) if b.size else None,
                                        _p(out), batch, m, k, n, int(bool(transA)),
                                        int(bool(transB))), "Gemm")
    return out


def Unary(kind: int, a, out=None) -> np.ndarray:
    """backend.Elementwiser.Unary on the device: out[i] = f_kind(a[i]) over host
    float64 data (kinds: _lib.GONN_UN_*, backend/backend.go:36-45). Raises on an
    unknown kind or a device error."""
    a = np.ascontiguousarray(a, dtype=np.float64).reshape(-1)
    if out is None:
        out = np.empty_like(a)
    elif not (isinstance(out, np.ndarray) and out.dtype == np.float64 and out.flags.c_contiguous
              and out.size == a.size):
        raise ValueError("Unary: out must be a contiguous float64 array of a's size")
    if a.size:
        check(_lib.load().gonn_hip_unary_f64(int(kind), _p(a), _p(out), a.size), "Unary")
    return out


def Binary(kind: int, a, b, out=None) -> np.ndarray:
    """backend.Elementwiser.Binary on the device: out[i] = a[i] op b[i] (kinds:
    _lib.GONN_BIN_*, backend/backend.go:51-58)."""
    a = np.ascontiguousarray(a, dtype=np.float64).reshape(-1)
    b = _f64(b, a.size, "Binary B").reshape(-1)
    if out is None:
        out = np.empty_like(a)
    elif not (isinstance(out, np.ndarray) and out.dtype == np.float64 and out.flags.c_contiguous
              and out.size == a.size):
        raise ValueError("Binary: out must be a contiguous float64 array of a's size")
    if a.size:
        check(_lib.load().gonn_hip_binary_f64(int(kind), _p(a), _p(b), _p(out), a.size), "Binary")
    return out


def BenchFlashAttnF64(BH: int, S: int, d: int, iters: int, causal: bool) -> float:
    """Device-resident, event-timed forward; mean ms per launch."""
    ms = float(_lib.load().gonn_hip_bench_flash_attn_f64(BH, S, d, iters, int(bool(causal))))
    if ms < 0:
        raise GonnHipError(int(ms), "BenchFlashAttnF64")
    return ms


def BenchFlashAttnF64Bwd(BH: int, S: int, d: int, iters: int, causal: bool) -> float:
    """New (the reference times no backward): the exact-mode (SetAttnMode
    "f64") backward, device-resident and event-timed like BenchFlashAttnF64;
    mean ms per call. Raises GonnHipError in any other mode."""
    ms = float(_lib.load().gonn_hip_bench_flash_attn_f64_bwd(BH, S, d, iters, int(bool(causal))))
    if ms < 0:
        raise GonnHipError(int(ms), "BenchFlashAttnF64Bwd")
    return ms


# ---------------------------------------------------------------------------
# device-resident API on torch tensors
# ---------------------------------------------------------------------------
def _torch():
    import torch  # imported lazily: the f64 API above does not need torch
    return torch


def _dtype_code(t):
    torch = _torch()
    if t.dtype == torch.float32:
        return GONN_F32
    if t.dtype == torch.bfloat16:
        return GONN_BF16
    if t.dtype == torch.int32:
        return GONN_I32
    if t.dtype == torch.float64:
        return _lib.GONN_F64
    raise TypeError(f"unsupported tensor dtype {t.dtype}")


def buf(t) -> Buf:
    if t is None:
        return Buf(None, 0, GONN_F32)
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("device API needs contiguous device tensors")
    return Buf(t.data_ptr(), t.numel() * t.element_size(), _dtype_code(t))


def _torch_stream(stream):
    return _torch().cuda.current_stream() if stream is None else stream


def _stream(stream):
    return ctypes.c_void_p(_torch_stream(stream).cuda_stream)


class _Workspace:
    """Grow-only device workspace per (device, stream). Each call uses it in
    stream order, so reuse across calls on one stream is safe."""

    def __init__(self):
        self._bufs = {}
        self._mu = threading.Lock()

    def get(self, nbytes: int, device, stream):
        """stream: the torch stream the call runs on. A new buffer is
        allocated on that stream, and a replaced one is marked as used there,
        so torch's caching allocator cannot hand it out while queued kernels
        still read it."""
        if nbytes == 0:
            return None
        torch = _torch()
        stream = _torch_stream(stream)
        key = (str(device), stream.cuda_stream)
        with self._mu:
            t = self._bufs.get(key)
            if t is None or t.numel() < nbytes:
                if t is not None:
                    t.record_stream(stream)
                with torch.cuda.stream(stream):
                    t = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
                self._bufs[key] = t
            return t


_WS = _Workspace()


def _shape4(t, name):
    if t.dim() == 4:
        return t.shape[0], t.shape[1], t.shape[2], t.shape[3]
    if t.dim() == 3:
        return t.shape[0], 1, t.shape[1], t.shape[2]
    raise ValueError(f"{name}: expected (B,H,S,D) or (BH,S,D), got {tuple(t.shape)}")


def mask_strides(shape, B: int, H: int, Sq: int, Sk: int):
    """expandAttnMask (nn/attention.go:242-257): the (sequence, head) element
    strides of an additive mask of shape (Sq,Sk), (B*H,Sq,Sk), (B,Sq,Sk) or
    (B,H,Sq,Sk); rows are Sk apart. Other shapes raise ValueError."""
    s = tuple(int(x) for x in shape)
    if s == (Sq, Sk):
        return 0, 0
    if s == (B * H, Sq, Sk) or s == (B, H, Sq, Sk):
        return H * Sq * Sk, Sq * Sk
    if s == (B, Sq, Sk):
        return Sq * Sk, 0
    raise ValueError(f"MultiHeadAttention: attn mask shape {list(s)} incompatible with "
                     f"(Tq,Tk)=({Sq},{Sk}), (B,Tq,Tk) B={B}, (B*H,Tq,Tk) B*H={B * H}, "
                     f"or (B,H,Tq,Tk)")


def attn_fwd(q, k, v, *, causal: bool = False, scale=None, mode="fp32", out=None,
             lse=True, lse_out=None, kv_len=None, stream=None, attn_mask=None):
    """O = softmax(scale QK^T + mask) V on device tensors.

    q (B,H,Sq,D) or (BH,Sq,D); k, v (.., Sk, D). fp32 mode needs float32
    inputs; bf16 mode takes float32 or bfloat16 inputs. Returns (O, LSE) with O
    float32 like q and LSE float32 (B*H, Sq) in natural-log units (or None when
    lse is False). out / lse_out may supply preallocated outputs. kv_len: an
    optional int32 device tensor (B,) of valid keys per sequence (prefix key
    padding; a 3-D q counts each slice as its own sequence). attn_mask: an
    optional float32 device tensor, the additive mask of WithAttnMask in one
    of mask_strides' shapes, added to the scores in the stated mode.
    """
    torch = _torch()
    B, H, Sq, D = _shape4(q, "q")
    Sk = k.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    l = lse_out
    if l is None and lse:
        l = torch.empty((B * H, Sq), dtype=torch.float32, device=q.device)
    mb, sb, sh = Buf(), 0, 0
    if attn_mask is not None:
        sb, sh = mask_strides(attn_mask.shape, B, H, Sq, Sk)
        mb = buf(attn_mask)
    a = FwdArgs(buf(q), buf(k), buf(v), buf(out), buf(l), B, H, Sq, Sk, D, float(scale),
                int(bool(causal)), MODES[mode], buf(kv_len) if kv_len is not None else Buf(),
                mb, sb, sh)
    lib = _lib.load()
    st = _stream(stream)
    nb = lib.gonn_hip_attn_workspace_bytes(GONN_OP_FWD, ctypes.byref(a))
    ws = _WS.get(nb, q.device, stream)
    check(lib.gonn_hip_attn_fwd(ctypes.byref(a), ws.data_ptr() if ws is not None else None,
                                nb, st), "attn_fwd")
    return out, l


def attn_bwd(q, k, v, o, lse, dO, *, causal: bool = False, scale=None, mode="fp32",
             out=None, stream=None, kv_len=None, attn_mask=None):
    """dQ, dK, dV (float32) from the saved forward tensors (all float32).
    out may supply preallocated (dq, dk, dv). kv_len: optional int32 (B,)
    device tensor, the key padding the forward was run with; attn_mask: its
    additive mask."""
    torch = _torch()
    B, H, S, D = _shape4(q, "q")
    Sk = k.shape[-2]  # key rows: != S for cross-attention
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        dq = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        dk, dv = (torch.empty(k.shape, dtype=torch.float32, device=q.device) for _ in range(2))
    else:
        dq, dk, dv = out
    mb, sb, sh = Buf(), 0, 0
    if attn_mask is not None:
        sb, sh = mask_strides(attn_mask.shape, B, H, S, Sk)
        mb = buf(attn_mask)
    a = BwdArgs(buf(q), buf(k), buf(v), buf(o), buf(lse), buf(dO), buf(dq), buf(dk), buf(dv),
                B, H, S, D, float(scale), int(bool(causal)), MODES[mode], 1,
                buf(kv_len) if kv_len is not None else Buf(None, 0, GONN_I32), mb, sb, sh,
                0 if Sk == S else Sk)
    lib = _lib.load()
    st = _stream(stream)
    nb = lib.gonn_hip_attn_workspace_bytes(GONN_OP_BWD, ctypes.byref(a))
    ws = _WS.get(nb, q.device, stream)
    check(lib.gonn_hip_attn_bwd(ctypes.byref(a), ws.data_ptr() if ws is not None else None,
                                nb, st), "attn_bwd")
    return dq, dk, dv


def attn_decode(q, kcache, vcache, kv_len, *, scale=None, split_keys: int = 0, out=None,
                stream=None):
    """Split-KV decode: q (B,H,D) float32/bfloat16, caches (B,H,Lmax,D) bfloat16,
    kv_len int32 (B,) on the device. Returns o (B,H,D) float32."""
    torch = _torch()
    B, H, Lmax, D = kcache.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float32, device=q.device)
    a = DecodeArgs(buf(q), buf(kcache), buf(vcache), buf(kv_len), buf(out), B, H, Lmax, D,
                   float(scale), int(split_keys))
    lib = _lib.load()
    st = _stream(stream)
    nb = lib.gonn_hip_attn_workspace_bytes(GONN_OP_DECODE, ctypes.byref(a))
    ws = _WS.get(nb, q.device, stream)
    check(lib.gonn_hip_attn_decode(ctypes.byref(a), ws.data_ptr() if ws is not None else None,
                                   nb, st), "attn_decode")
    return out


# ---------------------------------------------------------------------------
# KV cache (incremental decoding)
# ---------------------------------------------------------------------------
class KVCache:
    """One attention layer's device KV cache (gonn_hip_kvcache_*): bf16 K/V of
    B sequences x H heads, up to Lmax positions of head dim D, plus each
    sequence's length. New relative to the reference, which has no KV cache;
    attend() is ForwardMasked with a key-padding mask (nn/attention.go:305-341)
    over the cached positions of each sequence.

    Host fp64 methods (the cgo-style path): append_f64, attend_f64.
    Device methods on torch tensors: append, attend.
    """

    def __init__(self, B: int, H: int, Lmax: int, D: int):
        self.B, self.H, self.Lmax, self.D = int(B), int(H), int(Lmax), int(D)
        self._h = ctypes.c_void_p()
        check(_lib.load().gonn_hip_kvcache_create(ctypes.byref(self._h), self.B, self.H,
                                                  self.Lmax, self.D), "KVCache")

    def close(self) -> None:
        if self._h:
            check(_lib.load().gonn_hip_kvcache_free(self._h), "KVCache.close")
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _live(self):
        if not self._h:
            raise ValueError("KVCache: closed")
        return self._h

    def reset(self) -> None:
        check(_lib.load().gonn_hip_kvcache_reset(self._live()), "KVCache.reset")

    def lengths(self) -> np.ndarray:
        out = np.zeros(self.B, dtype=np.int32)
        check(_lib.load().gonn_hip_kvcache_lengths(
            self._live(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int))), "KVCache.lengths")
        return out

    def _counts(self, counts, T):
        if counts is None:
            return None, None
        c = np.ascontiguousarray(counts, dtype=np.int32)
        if c.shape != (self.B,):
            raise ValueError(f"KVCache: counts must have {self.B} entries")
        return c, c.ctypes.data_as(ctypes.POINTER(ctypes.c_int))

    def append_f64(self, k, v, counts=None) -> None:
        """k, v host (B,H,T,D) float64; sequence b takes its first counts[b]
        rows (all T when counts is None)."""
        k = np.ascontiguousarray(k, dtype=np.float64)
        v = np.ascontiguousarray(v, dtype=np.float64)
        if k.ndim != 4 or k.shape != v.shape or k.shape[:2] != (self.B, self.H) \
                or k.shape[3] != self.D:
            raise ValueError(f"KVCache.append_f64: k, v must be ({self.B},{self.H},T,{self.D})")
        c, cp = self._counts(counts, k.shape[2])
        check(_lib.load().gonn_hip_kvcache_append_f64(self._live(), _p(k), _p(v), k.shape[2],
                                                       cp), "KVCache.append_f64")

    def attend_f64(self, q, scale=None) -> np.ndarray:
        """q host (B,H,D) float64 -> o (B,H,D) float64."""
        q = np.ascontiguousarray(q, dtype=np.float64)
        if q.shape != (self.B, self.H, self.D):
            raise ValueError(f"KVCache.attend_f64: q must be ({self.B},{self.H},{self.D})")
        if scale is None:
            scale = 1.0 / math.sqrt(self.D)
        o = np.zeros_like(q)
        check(_lib.load().gonn_hip_kvcache_attend_f64(self._live(), _p(q), _p(o), float(scale)),
              "KVCache.attend_f64")
        return o

    def append(self, k, v, counts=None, stream=None) -> None:
        """k, v device (B,H,T,D) float32 or bfloat16 (both the same dtype)."""
        if k.dim() != 4 or tuple(k.shape) != tuple(v.shape):
            raise ValueError("KVCache.append: k, v must be (B,H,T,D) of the same shape")
        c, cp = self._counts(counts, k.shape[2])
        kb, vb = buf(k), buf(v)
        check(_lib.load().gonn_hip_kvcache_append(self._live(), ctypes.byref(kb),
                                                   ctypes.byref(vb), int(k.shape[2]), cp,
                                                   _stream(stream)), "KVCache.append")

    def attend(self, q, scale=None, out=None, stream=None):
        """q device (B,H,D) float32/bfloat16 -> o (B,H,D) float32."""
        torch = _torch()
        if scale is None:
            scale = 1.0 / math.sqrt(self.D)
        if out is None:
            out = torch.empty((self.B, self.H, self.D), dtype=torch.float32, device=q.device)
        qb, ob = buf(q), buf(out)
        check(_lib.load().gonn_hip_kvcache_attend(self._live(), ctypes.byref(qb),
                                                   ctypes.byref(ob), float(scale),
                                                   _stream(stream)), "KVCache.attend")
        return out

    def attend_causal_workspace_bytes(self, T: int) -> int:
        return int(_lib.load().gonn_hip_kvcache_attend_causal_workspace_bytes(self._live(), int(T)))

    def attend_causal(self, q, scale=None, out=None, ws=None, stream=None):
        """Causal multi-token attend: q device (B,H,T,D) float32, the queries of
        the last T cached positions of every sequence -> o (B,H,T,D) float32;
        query t sees cached positions [0, len_b - T + t]. New relative to the
        reference (no KV cache); equal to the rows of a top-left causal
        attention over each whole sequence (nn/attention.go:185-196)."""
        torch = _torch()
        if q.dim() != 4 or tuple(q.shape[:2]) != (self.B, self.H) or q.shape[3] != self.D:
            raise ValueError(f"KVCache.attend_causal: q must be ({self.B},{self.H},T,{self.D})")
        T = int(q.shape[2])
        if scale is None:
            scale = 1.0 / math.sqrt(self.D)
        if out is None:
            out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        need = self.attend_causal_workspace_bytes(T)
        if ws is None:
            ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        qb, ob = buf(q), buf(out)
        check(_lib.load().gonn_hip_kvcache_attend_causal(
            self._live(), ctypes.byref(qb), ctypes.byref(ob), T, float(scale),
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(stream)), "KVCache.attend_causal")
        return out


class DeviceMHA:
    """Device-resident multi-head attention (gonn_hip_mha_*): the forward of
    nn.MultiHeadAttention (nn/attention.go:107-148) with its four projections'
    weights in HBM. forward() takes host fp64 (B, T, *) arrays and makes one
    upload and one download per call; forward_dev() runs on torch float64
    device tensors with a caller workspace and allocates nothing.
    New relative to the reference, whose CUDA path copies across PCIe around
    every GEMM and around the fused core."""

    def __init__(self, E: int, H: int, Wq, bq, Wk, bk, Wv, bv, Wo, bo):
        E, H = int(E), int(H)
        Wq, Wo = _f64(Wq, E * E, "DeviceMHA Wq"), _f64(Wo, E * E, "DeviceMHA Wo")
        Wk = np.ascontiguousarray(Wk, dtype=np.float64)
        Wv = np.ascontiguousarray(Wv, dtype=np.float64)
        if Wk.ndim != 2 or Wk.shape[0] != E or Wv.ndim != 2 or Wv.shape[0] != E:
            raise ValueError("DeviceMHA: Wk and Wv must be (E, in)")
        self.E, self.H, self.kdim, self.vdim = E, H, int(Wk.shape[1]), int(Wv.shape[1])
        bs = [None if b is None else _f64(b, E, "DeviceMHA bias") for b in (bq, bk, bv, bo)]
        self._keep = (Wq, Wk, Wv, Wo, bs)
        self._h = ctypes.c_void_p()
        bp = [_p(b) if b is not None else None for b in bs]
        check(_lib.load().gonn_hip_mha_create(ctypes.byref(self._h), E, H, self.kdim, self.vdim,
                                              _p(Wq), bp[0], _p(Wk), bp[1], _p(Wv), bp[2],
                                              _p(Wo), bp[3]), "DeviceMHA")
        self._keep = None

    def close(self) -> None:
        if self._h:
            check(_lib.load().gonn_hip_mha_free(self._h), "DeviceMHA.close")
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _live(self):
        if not self._h:
            raise ValueError("DeviceMHA: closed")
        return self._h

    def _shapes(self, q, k, v):
        if q.ndim != 3 or q.shape[2] != self.E or k.ndim != 3 or k.shape[2] != self.kdim or \
                v.ndim != 3 or v.shape[2] != self.vdim or k.shape[:2] != v.shape[:2] or \
                k.shape[0] != q.shape[0]:
            raise ValueError(f"DeviceMHA: shapes q {tuple(q.shape)} k {tuple(k.shape)} "
                             f"v {tuple(v.shape)}")
        return q.shape[0], q.shape[1], k.shape[1]

    def forward(self, q, k, v, causal: bool = False, kv_len=None) -> np.ndarray:
        same_k, same_v = k is q, v is k
        q = np.ascontiguousarray(q, dtype=np.float64)
        k = q if same_k else np.ascontiguousarray(k, dtype=np.float64)
        v = k if same_v else np.ascontiguousarray(v, dtype=np.float64)
        B, Tq, Tk = self._shapes(q, k, v)
        out = np.empty((B, Tq, self.E))
        kl = None
        if kv_len is not None:
            kl = np.ascontiguousarray(kv_len, dtype=np.int32)
            if kl.shape != (B,):
                raise ValueError(f"DeviceMHA: kv_len must have {B} entries")
        check(_lib.load().gonn_hip_mha_forward_f64(
            self._live(), _p(q), _p(k), _p(v), _p(out), B, Tq, Tk, int(bool(causal)),
            kl.ctypes.data_as(ctypes.POINTER(ctypes.c_int)) if kl is not None else None),
            "DeviceMHA.forward")
        return out

    def workspace_bytes(self, B: int, Tq: int, Tk: int) -> int:
        return int(_lib.load().gonn_hip_mha_workspace_bytes(self._live(), B, Tq, Tk))

    def forward_dev(self, q, k, v, out=None, causal: bool = False, kv_len=None, ws=None):
        """q, k, v: contiguous torch float64 CUDA tensors; kv_len: int32 CUDA
        tensor or None; ws: a uint8 CUDA tensor of workspace_bytes() or None
        (then one is allocated by torch); runs on torch's current stream."""
        import torch
        B, Tq, Tk = self._shapes(q, k, v)
        for t in (q, k, v):
            if t.dtype != torch.float64 or not t.is_cuda or not t.is_contiguous():
                raise ValueError("DeviceMHA.forward_dev: inputs must be contiguous float64 CUDA tensors")
        if out is None:
            out = torch.empty((B, Tq, self.E), dtype=torch.float64, device=q.device)
        need = self.workspace_bytes(B, Tq, Tk)
        if ws is None:
            ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        kb = buf(kv_len) if kv_len is not None else None
        st = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
        check(_lib.load().gonn_hip_mha_forward_dev(
            self._live(), ctypes.byref(buf(q)), ctypes.byref(buf(k)), ctypes.byref(buf(v)),
            ctypes.byref(buf(out)), B, Tq, Tk, int(bool(causal)),
            ctypes.byref(kb) if kb is not None else None, ctypes.c_void_p(ws.data_ptr()),
            ws.numel(), st), "DeviceMHA.forward_dev")
        return out

    def incremental_workspace_bytes(self, cache: "KVCache", T: int) -> int:
        return int(_lib.load().gonn_hip_mha_incremental_workspace_bytes(
            self._live(), cache._live(), int(T)))

    def forward_incremental_dev(self, x, cache: "KVCache", out=None, ws=None):
        """Incremental self-attention on the device: x a contiguous torch
        float64 CUDA tensor (B, T, E) of T new positions per sequence; their
        K/V rows are appended to `cache` and out (B, T, E) float64 holds the
        last T rows of the causal forward over everything the cache holds.
        One host synchronisation per call; runs on torch's current stream.
        New relative to the reference (no KV cache)."""
        import torch
        if x.dim() != 3 or x.shape[2] != self.E or x.dtype != torch.float64 or not x.is_cuda \
                or not x.is_contiguous():
            raise ValueError(f"DeviceMHA.forward_incremental_dev: x must be a contiguous "
                             f"float64 CUDA tensor (B, T, {self.E})")
        B, T = int(x.shape[0]), int(x.shape[1])
        if B != cache.B:
            raise ValueError(f"DeviceMHA.forward_incremental_dev: cache holds {cache.B} sequences")
        need = self.incremental_workspace_bytes(cache, T)
        if need == 0:
            raise ValueError("DeviceMHA.forward_incremental_dev: cache and layer do not match "
                             "(cache must be (B, H, *, 64|128) of a self-attention layer)")
        if out is None:
            out = torch.empty((B, T, self.E), dtype=torch.float64, device=x.device)
        if ws is None:
            ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        st = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        check(_lib.load().gonn_hip_mha_forward_incremental_dev(
            self._live(), cache._live(), ctypes.byref(buf(x)), ctypes.byref(buf(out)), T,
            ctypes.c_void_p(ws.data_ptr()), ws.numel(), st), "DeviceMHA.forward_incremental_dev")
        return out


__all__ = ["Available", "Supports", "SetAttnMode", "AttnMode", "Version", "SelftestMFMA",
           "FlashAttnF64", "FlashAttnF64Fwd", "FlashAttnF64Bwd", "FlashAttnF64Ex",
           "FlashAttnF64BwdEx", "mask_strides", "Gemm",
           "Unary", "Binary",
           "BenchFlashAttnF64", "BenchFlashAttnF64Bwd", "attn_fwd", "attn_bwd", "attn_decode",
           "KVCache", "DeviceMHA", "buf", "GonnHipError"]
