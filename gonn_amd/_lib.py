"""ctypes binding of libgonn_hip.so (the C ABI in include/gonn_hip.h).

This is the Python counterpart of the cgo block a Go maintainer adds in
backend/hip (the reference's backend/cuda/cuda.go:1-20 pattern). It loads the
in-tree library and fails loudly when it has not been built: there is no CPU
fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgonn_hip.so")

# error codes (include/gonn_hip.h)
GONN_OK = 0
GONN_E_INVALID = -1
GONN_E_UNSUPPORTED = -2
GONN_E_WORKSPACE = -3
GONN_E_NOMEM = -4
GONN_E_NODEVICE = -5
GONN_E_INJECTED = -6
GONN_E_BLAS = -7

GONN_F32, GONN_BF16, GONN_F64, GONN_I32 = 0, 1, 2, 3
GONN_ATTN_FP32_MFMA, GONN_ATTN_BF16_MFMA, GONN_ATTN_FP64 = 0, 1, 2
# backend.UnaryKind / BinaryKind values (backend/backend.go:26-58): a shared ABI.
(GONN_UN_RELU, GONN_UN_SIGMOID, GONN_UN_TANH, GONN_UN_EXP, GONN_UN_LOG, GONN_UN_GELU,
 GONN_UN_SILU, GONN_UN_GELU_EXACT) = range(8)
GONN_BIN_ADD, GONN_BIN_SUB, GONN_BIN_MUL, GONN_BIN_DIV = range(4)
GONN_OP_FWD, GONN_OP_BWD, GONN_OP_DECODE = 0, 1, 2

# Every symbol include/gonn_hip.h declares.
EXPORTED_SYMBOLS = (
    "gonn_hip_version", "gonn_hip_strerror", "gonn_hip_available", "gonn_hip_attn_supports",
    "gonn_hip_set_attn_mode", "gonn_hip_get_attn_mode", "gonn_hip_attn_workspace_bytes",
    "gonn_hip_attn_fwd", "gonn_hip_attn_bwd", "gonn_hip_attn_decode", "gonn_hip_alloc",
    "gonn_hip_free", "gonn_hip_upload_from_f64", "gonn_hip_download_to_f64",
    "gonn_hip_memcpy_h2d", "gonn_hip_memcpy_d2h", "gonn_hip_stream_sync",
    "gonn_hip_flash_attn_f64", "gonn_hip_flash_attn_f64_fwd", "gonn_hip_flash_attn_f64_bwd",
    "gonn_hip_bench_flash_attn_f64", "gonn_hip_bench_flash_attn_f64_bwd",
    "gonn_hip_profile_enable", "gonn_hip_profile_reset", "gonn_hip_profile_read", "gonn_hip_selftest_mfma",
    "gonn_hip_kvcache_create", "gonn_hip_kvcache_free", "gonn_hip_kvcache_reset",
    "gonn_hip_kvcache_lengths", "gonn_hip_kvcache_append", "gonn_hip_kvcache_append_f64",
    "gonn_hip_kvcache_attend", "gonn_hip_kvcache_attend_f64", "gonn_hip_flash_attn_f64_ex",
    "gonn_hip_gemm_f64", "gonn_hip_gemm_f64_dev",
    "gonn_hip_unary_f64", "gonn_hip_binary_f64", "gonn_hip_unary_f64_dev", "gonn_hip_binary_f64_dev",
    "gonn_hip_mha_create", "gonn_hip_mha_free", "gonn_hip_mha_forward_f64",
    "gonn_hip_mha_workspace_bytes", "gonn_hip_mha_forward_dev", "gonn_hip_flash_attn_f64_bwd_ex",
    "gonn_hip_flash_attn_f64_masked", "gonn_hip_flash_attn_f64_bwd_masked",
    "gonn_hip_attn_decode_noalloc",
    "gonn_hip_kvcache_attend_causal_workspace_bytes", "gonn_hip_kvcache_attend_causal",
    "gonn_hip_mha_incremental_workspace_bytes", "gonn_hip_mha_forward_incremental_dev",
    "gonn_hip_calib_mfma", "gonn_hip_calib_clock_start", "gonn_hip_calib_clock_read",
)

# Size of the library-owned scratch array of gonn_hip_attn_decode_noalloc
# (GONN_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 << 20


class GonnHipError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, code: int, where: str):
        self.code = int(code)
        msg = strerror(code) if _lib is not None else str(code)
        super().__init__(f"{where}: {msg} (code {code})")


class Buf(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_size_t), ("dtype", ctypes.c_int)]


class FwdArgs(ctypes.Structure):
    _fields_ = [("q", Buf), ("k", Buf), ("v", Buf), ("o", Buf), ("lse", Buf),
                ("B", ctypes.c_int), ("H", ctypes.c_int), ("Sq", ctypes.c_int),
                ("Sk", ctypes.c_int), ("D", ctypes.c_int), ("scale", ctypes.c_double),
                ("causal", ctypes.c_int), ("mode", ctypes.c_int), ("kv_len", Buf),
                ("attn_mask", Buf), ("mask_stride_b", ctypes.c_int64),
                ("mask_stride_h", ctypes.c_int64)]


class BwdArgs(ctypes.Structure):
    _fields_ = [("q", Buf), ("k", Buf), ("v", Buf), ("o", Buf), ("lse", Buf), ("dO", Buf),
                ("dq", Buf), ("dk", Buf), ("dv", Buf),
                ("B", ctypes.c_int), ("H", ctypes.c_int), ("S", ctypes.c_int),
                ("D", ctypes.c_int), ("scale", ctypes.c_double), ("causal", ctypes.c_int),
                ("mode", ctypes.c_int), ("deterministic", ctypes.c_int), ("kv_len", Buf),
                ("attn_mask", Buf), ("mask_stride_b", ctypes.c_int64),
                ("mask_stride_h", ctypes.c_int64), ("Sk", ctypes.c_int)]


class DecodeArgs(ctypes.Structure):
    _fields_ = [("q", Buf), ("kcache", Buf), ("vcache", Buf), ("kv_len", Buf), ("o", Buf),
                ("B", ctypes.c_int), ("H", ctypes.c_int), ("Lmax", ctypes.c_int),
                ("D", ctypes.c_int), ("scale", ctypes.c_double), ("split_keys", ctypes.c_int)]


_lib = None


def load() -> ctypes.CDLL:
    """Load the in-tree library; raise if it is missing (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m gonn_amd.build` (hipcc, gfx950). "
            "gonn_amd has no CPU fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    dp = ctypes.POINTER(ctypes.c_double)
    vp = ctypes.c_void_p
    sz = ctypes.c_size_t
    i = ctypes.c_int
    lib.gonn_hip_version.restype = ctypes.c_char_p
    lib.gonn_hip_strerror.restype = ctypes.c_char_p
    lib.gonn_hip_strerror.argtypes = [i]
    lib.gonn_hip_available.restype = i
    lib.gonn_hip_attn_supports.argtypes = [i, i, i]
    lib.gonn_hip_set_attn_mode.argtypes = [i]
    lib.gonn_hip_attn_workspace_bytes.restype = sz
    lib.gonn_hip_attn_workspace_bytes.argtypes = [i, vp]
    lib.gonn_hip_attn_fwd.argtypes = [ctypes.POINTER(FwdArgs), vp, sz, vp]
    lib.gonn_hip_attn_bwd.argtypes = [ctypes.POINTER(BwdArgs), vp, sz, vp]
    lib.gonn_hip_attn_decode.argtypes = [ctypes.POINTER(DecodeArgs), vp, sz, vp]
    lib.gonn_hip_attn_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), vp]
    lib.gonn_hip_alloc.argtypes = [ctypes.POINTER(Buf), sz, i]
    lib.gonn_hip_free.argtypes = [ctypes.POINTER(Buf)]
    lib.gonn_hip_upload_from_f64.argtypes = [ctypes.POINTER(Buf), dp, sz, vp]
    lib.gonn_hip_download_to_f64.argtypes = [dp, ctypes.POINTER(Buf), sz, vp]
    lib.gonn_hip_memcpy_h2d.argtypes = [vp, vp, sz, vp]
    lib.gonn_hip_memcpy_d2h.argtypes = [vp, vp, sz, vp]
    lib.gonn_hip_stream_sync.argtypes = [vp]
    lib.gonn_hip_flash_attn_f64.argtypes = [dp, dp, dp, dp, i, i, i, ctypes.c_double, i]
    lib.gonn_hip_flash_attn_f64_fwd.argtypes = [dp, dp, dp, dp, dp, i, i, i, ctypes.c_double, i]
    lib.gonn_hip_flash_attn_f64_bwd.argtypes = [dp] * 9 + [i, i, i, ctypes.c_double, i]
    lib.gonn_hip_bench_flash_attn_f64.restype = ctypes.c_double
    lib.gonn_hip_bench_flash_attn_f64.argtypes = [i, i, i, i, i]
    lib.gonn_hip_bench_flash_attn_f64_bwd.restype = ctypes.c_double
    lib.gonn_hip_bench_flash_attn_f64_bwd.argtypes = [i, i, i, i, i]
    lib.gonn_hip_selftest_mfma.restype = i
    lib.gonn_hip_profile_enable.argtypes = [i]
    lib.gonn_hip_profile_read.argtypes = [ctypes.c_char_p, dp, ctypes.POINTER(i)]
    lib.gonn_hip_calib_mfma.argtypes = [i, dp, dp]
    lib.gonn_hip_calib_clock_start.argtypes = [ctypes.c_double, vp]
    lib.gonn_hip_calib_clock_read.argtypes = [dp]
    ip = ctypes.POINTER(i)
    lib.gonn_hip_kvcache_create.argtypes = [ctypes.POINTER(vp), i, i, i, i]
    lib.gonn_hip_kvcache_free.argtypes = [vp]
    lib.gonn_hip_kvcache_reset.argtypes = [vp]
    lib.gonn_hip_kvcache_lengths.argtypes = [vp, ip]
    lib.gonn_hip_kvcache_append.argtypes = [vp, ctypes.POINTER(Buf), ctypes.POINTER(Buf), i, ip, vp]
    lib.gonn_hip_kvcache_append_f64.argtypes = [vp, dp, dp, i, ip]
    lib.gonn_hip_kvcache_attend.argtypes = [vp, ctypes.POINTER(Buf), ctypes.POINTER(Buf),
                                            ctypes.c_double, vp]
    lib.gonn_hip_kvcache_attend_f64.argtypes = [vp, dp, dp, ctypes.c_double]
    lib.gonn_hip_flash_attn_f64_ex.argtypes = [dp, dp, dp, dp, dp, i, i, i, i, i, ctypes.c_double,
                                               i, ip]
    lib.gonn_hip_gemm_f64.argtypes = [dp, dp, dp, i, i, i, i, i, i]
    lib.gonn_hip_gemm_f64_dev.argtypes = [ctypes.POINTER(Buf), ctypes.POINTER(Buf),
                                          ctypes.POINTER(Buf), i, i, i, i, i, i, vp]
    lg = ctypes.c_long
    lib.gonn_hip_unary_f64.argtypes = [i, dp, dp, lg]
    lib.gonn_hip_binary_f64.argtypes = [i, dp, dp, dp, lg]
    lib.gonn_hip_unary_f64_dev.argtypes = [i, ctypes.POINTER(Buf), ctypes.POINTER(Buf), lg, vp]
    lib.gonn_hip_binary_f64_dev.argtypes = [i, ctypes.POINTER(Buf), ctypes.POINTER(Buf),
                                            ctypes.POINTER(Buf), lg, vp]
    lib.gonn_hip_flash_attn_f64_bwd_ex.argtypes = [dp] * 9 + [i, i, i, i, ctypes.c_double, i, ip]
    lg_ = ctypes.c_long
    lib.gonn_hip_flash_attn_f64_masked.argtypes = [dp] * 5 + [i] * 5 + [ctypes.c_double, i, ip,
                                                                        dp, lg_, lg_]
    lib.gonn_hip_flash_attn_f64_bwd_masked.argtypes = [dp] * 9 + [i] * 5 + [ctypes.c_double, i,
                                                                            ip, dp, lg_, lg_]
    lib.gonn_hip_mha_create.argtypes = [ctypes.POINTER(vp), i, i, i, i] + [dp] * 8
    lib.gonn_hip_mha_free.argtypes = [vp]
    lib.gonn_hip_mha_forward_f64.argtypes = [vp, dp, dp, dp, dp, i, i, i, i, ip]
    lib.gonn_hip_mha_workspace_bytes.argtypes = [vp, i, i, i]
    lib.gonn_hip_mha_workspace_bytes.restype = ctypes.c_size_t
    lib.gonn_hip_mha_forward_dev.argtypes = [vp] + [ctypes.POINTER(Buf)] * 4 + [i, i, i, i, ctypes.POINTER(Buf), vp, ctypes.c_size_t, vp]
    lib.gonn_hip_kvcache_attend_causal_workspace_bytes.restype = sz
    lib.gonn_hip_kvcache_attend_causal_workspace_bytes.argtypes = [vp, i]
    lib.gonn_hip_kvcache_attend_causal.argtypes = [vp, ctypes.POINTER(Buf), ctypes.POINTER(Buf), i,
                                                   ctypes.c_double, vp, sz, vp]
    lib.gonn_hip_mha_incremental_workspace_bytes.restype = sz
    lib.gonn_hip_mha_incremental_workspace_bytes.argtypes = [vp, vp, i]
    lib.gonn_hip_mha_forward_incremental_dev.argtypes = [vp, vp, ctypes.POINTER(Buf),
                                                         ctypes.POINTER(Buf), i, vp, sz, vp]
    _lib = lib
    return lib


def strerror(code: int) -> str:
    return load().gonn_hip_strerror(int(code)).decode()


def check(rc: int, where: str) -> None:
    if rc != 0:
        raise GonnHipError(rc, where)
