"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments with the documented codes before
touching the device. Also the host-side failure paths: a missing device or an
injected allocation failure raises (no silent CPU fallback)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import gonn_amd
from gonn_amd import _lib, hip
from gonn_amd._lib import (GONN_BF16, GONN_E_INJECTED, GONN_E_INVALID, GONN_E_NODEVICE,
                           GONN_E_UNSUPPORTED, GONN_E_WORKSPACE, GONN_F32, GONN_I32, GONN_OP_BWD,
                           GONN_OP_DECODE, GONN_OP_FWD, Buf, BwdArgs, DecodeArgs, FwdArgs)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gonn_hip.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(gonn_hip_\w+)\s*\(", txt)))


def test_header_symbols_are_exported():
    lib = _lib.load()
    decl = _declared()
    assert len(decl) >= 20
    assert sorted(_lib.EXPORTED_SYMBOLS) == decl
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if line.strip()}
    missing = [s for s in decl if s not in exported]
    assert not missing, missing
    for s in decl:
        assert getattr(lib, s) is not None


def test_library_is_built_for_gfx950_only():
    """The embedded offload bundle of our own build names gfx950 and no other
    GPU target."""
    data = open(_lib.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}, targets


def test_version_strerror_modes():
    assert "gfx950" in hip.Version()
    assert "invalid" in _lib.strerror(GONN_E_INVALID)
    assert "unsupported" in _lib.strerror(GONN_E_UNSUPPORTED)
    assert "workspace" in _lib.strerror(GONN_E_WORKSPACE)
    lib = _lib.load()
    assert lib.gonn_hip_set_attn_mode(7) == GONN_E_INVALID
    hip.SetAttnMode("bf16")
    assert hip.AttnMode() == "bf16"
    hip.SetAttnMode("f64")  # the f64 entry points' exact mode
    assert hip.AttnMode() == "f64" and lib.gonn_hip_get_attn_mode() == 2
    hip.SetAttnMode("fp32")
    assert hip.AttnMode() == "fp32"


@pytest.mark.parametrize("mode", ["bf16", "f64"])
def test_mode_from_environment(mode):
    code = "from gonn_amd import hip; print(hip.AttnMode())"
    env = dict(os.environ, GONN_HIP_ATTN_MODE=mode, PYTHONPATH=ROOT)
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         check=True)
    assert out.stdout.strip() == mode


def test_supports_gate():
    assert hip.Supports(64, 128, 128) and hip.Supports(128, 1, 4096)
    assert hip.Supports(64, 100, 300)  # Tq != Tk is covered (top-left causal)
    assert not hip.Supports(96, 128, 128)
    assert not hip.Supports(64, 0, 128)


# fake device pointers: the checks below must fail before any device access
P = 0x10000


def _fwd_args(**kw):
    B, H, Sq, Sk, D = kw.get("B", 2), kw.get("H", 3), kw.get("Sq", 64), kw.get("Sk", 64), \
        kw.get("D", 64)
    nq, nk = B * H * Sq * D * 4, B * H * Sk * D * 4
    a = FwdArgs(Buf(P, nq, GONN_F32), Buf(P, nk, GONN_F32), Buf(P, nk, GONN_F32),
                Buf(P, nq, GONN_F32), Buf(None, 0, GONN_F32), B, H, Sq, Sk, D, 0.125,
                1, kw.get("mode", 0))
    return a


def _fwd(a, ws=None, nb=0):
    return _lib.load().gonn_hip_attn_fwd(ctypes.byref(a), ws, nb, None)


def test_fwd_argument_errors():
    a = _fwd_args(D=96)
    assert _fwd(a) == GONN_E_UNSUPPORTED
    a = _fwd_args(Sq=0)
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args(mode=5)
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args(mode=2)  # the f64 entries' exact mode is not a device-entry mode
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args()
    a.q.ptr = None
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args()
    a.k.bytes -= 4  # short buffer
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args()
    a.o.dtype = GONN_BF16  # O must be f32
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args()
    a.q.dtype = GONN_BF16  # fp32 mode needs f32 operands
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args()
    a.scale = float("nan")
    assert _fwd(a) == GONN_E_INVALID
    a = _fwd_args()
    a.lse = Buf(P, 4, GONN_F32)  # too short for (B*H, Sq)
    assert _fwd(a) == GONN_E_INVALID
    assert _lib.load().gonn_hip_attn_fwd(None, None, 0, None) == GONN_E_INVALID


def test_fwd_workspace_contract():
    lib = _lib.load()
    a = _fwd_args(mode=0)
    assert lib.gonn_hip_attn_workspace_bytes(GONN_OP_FWD, ctypes.byref(a)) == 0
    a = _fwd_args(mode=1, B=1, H=2, Sk=100, D=128)
    nb = lib.gonn_hip_attn_workspace_bytes(GONN_OP_FWD, ctypes.byref(a))
    assert nb >= 2 * 2 * 128 * 128 * 2  # Kb + Vt, keys padded to 128
    assert _fwd(a) == GONN_E_WORKSPACE
    assert _fwd(a, P, nb - 1) == GONN_E_WORKSPACE


def test_decode_argument_errors():
    lib = _lib.load()
    B, H, L, D = 2, 2, 256, 128
    mk = lambda: DecodeArgs(Buf(P, B * H * D * 2, GONN_BF16),  # noqa: E731
                            Buf(P, B * H * L * D * 2, GONN_BF16),
                            Buf(P, B * H * L * D * 2, GONN_BF16), Buf(P, B * 4, GONN_I32),
                            Buf(P, B * H * D * 4, GONN_F32), B, H, L, D, 0.088, 0)
    a = mk()
    nb = lib.gonn_hip_attn_workspace_bytes(GONN_OP_DECODE, ctypes.byref(a))
    assert nb > 0
    assert lib.gonn_hip_attn_decode(ctypes.byref(a), None, 0, None) == GONN_E_WORKSPACE
    a = mk()
    a.split_keys = 100
    assert lib.gonn_hip_attn_decode(ctypes.byref(a), P, nb, None) == GONN_E_INVALID
    a = mk()
    a.kcache.dtype = GONN_F32
    assert lib.gonn_hip_attn_decode(ctypes.byref(a), P, nb, None) == GONN_E_INVALID
    a = mk()
    a.kv_len.dtype = GONN_F32
    assert lib.gonn_hip_attn_decode(ctypes.byref(a), P, nb, None) == GONN_E_INVALID
    a = mk()
    a.D = 80
    assert lib.gonn_hip_attn_decode(ctypes.byref(a), P, nb, None) == GONN_E_UNSUPPORTED


def test_decode_noalloc_argument_errors():
    """The no-allocation decode checks its arguments like the workspace entry
    and rejects a call whose partials exceed the library's scratch array, all
    before any device access."""
    lib = _lib.load()
    B, H, L, D = 2, 2, 256, 128
    mk = lambda: DecodeArgs(Buf(P, B * H * D * 2, GONN_BF16),  # noqa: E731
                            Buf(P, B * H * L * D * 2, GONN_BF16),
                            Buf(P, B * H * L * D * 2, GONN_BF16), Buf(P, B * 4, GONN_I32),
                            Buf(P, B * H * D * 4, GONN_F32), B, H, L, D, 0.088, 0)
    assert lib.gonn_hip_attn_decode_noalloc(None, None) == GONN_E_INVALID
    a = mk()
    a.split_keys = 100
    assert lib.gonn_hip_attn_decode_noalloc(ctypes.byref(a), None) == GONN_E_INVALID
    a = mk()
    a.D = 80
    assert lib.gonn_hip_attn_decode_noalloc(ctypes.byref(a), None) == GONN_E_UNSUPPORTED
    # 2048 x 256 (b,h) slices of 16 splits at D=128 need 2048*256*16*130*4 B > 32 MiB.
    Bb, Hb, Lb = 2048, 256, 8192
    big = DecodeArgs(Buf(P, Bb * Hb * D * 2, GONN_BF16), Buf(P, Bb * Hb * Lb * D * 2, GONN_BF16),
                     Buf(P, Bb * Hb * Lb * D * 2, GONN_BF16), Buf(P, Bb * 4, GONN_I32),
                     Buf(P, Bb * Hb * D * 4, GONN_F32), Bb, Hb, Lb, D, 0.088, 0)
    need = lib.gonn_hip_attn_workspace_bytes(GONN_OP_DECODE, ctypes.byref(big))
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    assert lib.gonn_hip_attn_decode_noalloc(ctypes.byref(big), None) == GONN_E_WORKSPACE


def test_bwd_argument_errors():
    lib = _lib.load()
    B, H, S, D = 1, 2, 64, 64
    n = B * H * S * D * 4
    f = lambda: Buf(P, n, GONN_F32)  # noqa: E731
    a = BwdArgs(f(), f(), f(), f(), Buf(P, B * H * S * 4, GONN_F32), f(), f(), f(), f(), B, H,
                S, D, 0.125, 1, 0, 1)
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_WORKSPACE
    a.D = 48
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_UNSUPPORTED
    a.D = D
    a.lse.bytes = 8
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_INVALID
    a.lse.bytes = B * H * S * 4
    a.dq.dtype = GONN_BF16
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_INVALID
    a.dq.dtype = GONN_F32
    # Cross-attention: k, v, dk, dv must hold (B*H, Sk, D); a negative Sk is invalid.
    a.Sk = -1
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_INVALID
    a.Sk = 2 * S
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_INVALID
    for name in ("k", "v", "dk", "dv"):
        getattr(a, name).bytes = 2 * n
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_WORKSPACE
    # An additive mask must cover (B-1)*sb + (H-1)*sh + S*Sk f32 elements.
    a.attn_mask = Buf(P, 4 * S * 2 * S - 4, GONN_F32)
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_INVALID
    a.attn_mask.bytes = 4 * S * 2 * S
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_WORKSPACE
    a.mask_stride_h = -1
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), None, 0, None) == GONN_E_INVALID
    assert lib.gonn_hip_attn_workspace_bytes(GONN_OP_BWD, None) == 0


def test_bwd_workspace_contract():
    """fp32 mode needs LSE*log2(e) and D_i rows (BH, Sp) in f32; bf16 mode adds
    five packed bf16 operands (Q, dO, K, V rows and K^T; BH x Sp x D each),
    with Sp = S rounded up to 128."""
    lib = _lib.load()
    B, H, S, D = 1, 2, 200, 128
    n = B * H * S * D * 4
    f = lambda: Buf(P, n, GONN_F32)  # noqa: E731
    a = BwdArgs(f(), f(), f(), f(), Buf(P, B * H * S * 4, GONN_F32), f(), f(), f(), f(), B, H,
                S, D, 0.125, 1, 0, 1)
    Sp = 256
    nb32 = lib.gonn_hip_attn_workspace_bytes(GONN_OP_BWD, ctypes.byref(a))
    assert nb32 >= 2 * B * H * Sp * 4
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), P, nb32 - 1, None) == GONN_E_WORKSPACE
    a.mode = 1
    nb16 = lib.gonn_hip_attn_workspace_bytes(GONN_OP_BWD, ctypes.byref(a))
    assert nb16 >= nb32 + 5 * B * H * Sp * D * 2
    assert lib.gonn_hip_attn_bwd(ctypes.byref(a), P, nb32, None) == GONN_E_WORKSPACE


def test_bwd_ds_budget_workspace(monkeypatch):
    """The bf16 backward's stored dS is capped by a byte budget
    (GONN_HIP_BWD_DS_MB; 16 GiB by default): a call whose whole dS exceeds it
    runs its 128-key blocks in chunks that fit, at least one block each, and
    its workspace holds the largest chunk. B=2 H=2 S=4096 causal: key block kb
    reaches query tiles 2 kb .. 63, 64 - 2 kb blocks of 128 keys x 64 queries
    (16 KB) per slice, 1056 in all."""
    lib = _lib.load()
    B, H, S, D = 2, 2, 4096, 128
    n = B * H * S * D * 4
    f = lambda: Buf(P, n, GONN_F32)  # noqa: E731
    a = BwdArgs(f(), f(), f(), f(), Buf(P, B * H * S * 4, GONN_F32), f(), f(), f(), f(), B, H,
                S, D, 0.125, 1, 0, 1)
    a.mode = 1
    blk = 128 * 64 * 2 * B * H  # one block in every slice

    def ws(mb=None, dq=None):
        for k, v in (("GONN_HIP_BWD_DS_MB", mb), ("GONN_HIP_BWD_DQ", dq)):
            if v is None:
                monkeypatch.delenv(k, raising=False)
            else:
                monkeypatch.setenv(k, v)
        return lib.gonn_hip_attn_workspace_bytes(GONN_OP_BWD, ctypes.byref(a))
    full, recompute = ws(), ws(dq="recompute")
    assert full - recompute == 1056 * blk
    # 1 MB: one key block per chunk; key block 0 is the largest (64 blocks)
    assert ws("1") - recompute == 64 * blk
    # 20 MB: at most 320 blocks per slice; the chunks are key blocks 0-4
    # (64 + ... + 56 = 300), 5-10 (294), 11-19 (42 + ... + 26 = 306), 20-31
    # (156); the workspace holds the largest, 306
    assert ws("20") - recompute == 306 * blk
    assert ws("100") == full
    # By default (a 16 GiB budget) a call takes at most two chunks, else the
    # recompute path (O(S) memory): B=1 H=16 S=32768 causal stores 17.2 GB
    # of dS (two chunks), S=65536 69 GB (five).
    a.B, a.H, a.S = 1, 16, 32768
    a.dq = a.dk = a.dv = a.q = a.k = a.v = a.o = a.dO = Buf(P, 16 * 32768 * 128 * 4, GONN_F32)
    a.lse = Buf(P, 16 * 32768 * 4, GONN_F32)
    assert ws() > ws(dq="recompute") + 8 * 2**30
    a.S = 65536
    a.dq = a.dk = a.dv = a.q = a.k = a.v = a.o = a.dO = Buf(P, 16 * 65536 * 128 * 4, GONN_F32)
    a.lse = Buf(P, 16 * 65536 * 4, GONN_F32)
    assert ws() == ws(dq="recompute")
    assert ws("4096") > ws(dq="recompute")  # a given budget always chunks
    monkeypatch.delenv("GONN_HIP_BWD_DS_MB", raising=False)
    monkeypatch.delenv("GONN_HIP_BWD_DQ", raising=False)


def test_no_device_fails_loudly():
    """Without a gfx950 device the reference-named entry points raise; there is
    no CPU fallback (like the reference's non-cuda stubs,
    nn/flashattn_nocuda.go:12-20)."""
    if hip.Available():
        pytest.skip("a device is present")
    BH, S, d = 1, 4, 8
    x = np.zeros(BH * S * d)
    with pytest.raises(gonn_amd.GonnHipError) as e:
        hip.FlashAttnF64(x, x, x, np.zeros_like(x), BH, S, d, 0.35, True)
    assert e.value.code == GONN_E_NODEVICE
    with pytest.raises(gonn_amd.GonnHipError):
        hip.FlashAttnF64Fwd(x, x, x, BH, S, d, 0.35, True)
    with pytest.raises(gonn_amd.GonnHipError):
        hip.FlashAttnF64Bwd(x, x, x, x, np.zeros(BH * S), x, BH, S, d, 0.35, True)
    assert hip.BenchFlashAttnF64.__name__  # exists
    with pytest.raises(gonn_amd.GonnHipError):
        hip.BenchFlashAttnF64(BH, S, d, 3, True)
    from gonn_amd import nn
    assert not nn.fused_attn_available()
    E, H = 16, 2
    w = [np.eye(E), np.zeros(E)] * 4
    m = nn.MultiHeadAttention(E, H, *w)
    with pytest.raises(RuntimeError):
        m.forward(np.zeros((1, 3, E)), np.zeros((1, 3, E)), np.zeros((1, 3, E)), True)


def test_shim_argument_errors():
    lib = _lib.load()
    dp = ctypes.POINTER(ctypes.c_double)
    x = np.zeros(16)
    p = x.ctypes.data_as(dp)
    assert lib.gonn_hip_flash_attn_f64(p, p, p, p, 1, 2, 129, 0.1, 0) == GONN_E_INVALID
    assert lib.gonn_hip_flash_attn_f64(p, p, p, p, 0, 2, 8, 0.1, 0) == GONN_E_INVALID
    assert lib.gonn_hip_flash_attn_f64(None, p, p, p, 1, 2, 8, 0.1, 0) == GONN_E_INVALID
    assert lib.gonn_hip_bench_flash_attn_f64(1, 2, 8, 0, 0) < 0
    assert lib.gonn_hip_bench_flash_attn_f64_bwd(1, 2, 8, 0, 0) < 0


def test_injected_allocation_failure():
    code = ("import ctypes; from gonn_amd import _lib; from gonn_amd._lib import Buf;"
            "b = Buf(None, 0, 0); print(_lib.load().gonn_hip_alloc(ctypes.byref(b), 16, 0))")
    env = dict(os.environ, GONN_HIP_FAIL_ALLOC="1", PYTHONPATH=ROOT)
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         check=True)
    assert int(out.stdout.strip()) == GONN_E_INJECTED


def test_bench_refuses_multi_gpu():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True)
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_kvcache_argument_and_device_checks():
    """Bad arguments are rejected before the device is touched; with no gfx950
    device, creating a cache fails with GONN_E_NODEVICE (no CPU fallback)."""
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.gonn_hip_kvcache_create(None, 1, 1, 8, 64) == GONN_E_INVALID
    assert lib.gonn_hip_kvcache_create(ctypes.byref(h), 0, 1, 8, 64) == GONN_E_INVALID
    assert lib.gonn_hip_kvcache_create(ctypes.byref(h), 1, 1, 0, 64) == GONN_E_INVALID
    assert lib.gonn_hip_kvcache_create(ctypes.byref(h), 1, 1, 8, 96) == GONN_E_UNSUPPORTED
    assert not h.value
    assert lib.gonn_hip_kvcache_free(None) == 0
    assert lib.gonn_hip_kvcache_reset(None) == GONN_E_INVALID
    assert lib.gonn_hip_kvcache_lengths(None, None) == GONN_E_INVALID
    assert lib.gonn_hip_kvcache_append_f64(None, None, None, 1, None) == GONN_E_INVALID
    assert lib.gonn_hip_kvcache_attend_f64(None, None, None, 1.0) == GONN_E_INVALID
    if not hip.Available():
        assert lib.gonn_hip_kvcache_create(ctypes.byref(h), 1, 1, 8, 64) == GONN_E_NODEVICE
        assert not h.value
        with pytest.raises(hip.GonnHipError) as ei:
            hip.KVCache(1, 1, 8, 64)
        assert ei.value.code == GONN_E_NODEVICE


def test_mha_handle_argument_checks():
    import ctypes
    from gonn_amd import hip
    lib = _lib.load()
    h = ctypes.c_void_p()
    dp = ctypes.POINTER(ctypes.c_double)
    w = np.zeros(64 * 64)
    p = w.ctypes.data_as(dp)
    assert lib.gonn_hip_mha_create(None, 64, 4, 64, 64, p, None, p, None, p, None, p, None) == _lib.GONN_E_INVALID
    assert lib.gonn_hip_mha_create(ctypes.byref(h), 66, 4, 64, 64, p, None, p, None, p, None, p, None) == _lib.GONN_E_INVALID
    assert lib.gonn_hip_mha_create(ctypes.byref(h), 64, 4, 64, 64, None, None, p, None, p, None, p, None) == _lib.GONN_E_INVALID
    assert lib.gonn_hip_mha_create(ctypes.byref(h), 512, 2, 64, 64, p, None, p, None, p, None, p, None) == _lib.GONN_E_UNSUPPORTED
    assert lib.gonn_hip_mha_free(None) == 0
    assert lib.gonn_hip_mha_workspace_bytes(None, 1, 1, 1) == 0
    assert lib.gonn_hip_mha_forward_f64(None, p, p, p, p, 1, 1, 1, 0, None) == _lib.GONN_E_INVALID
    if not hip.Available():
        assert lib.gonn_hip_mha_create(ctypes.byref(h), 64, 4, 64, 64, p, None, p, None, p, None, p, None) == _lib.GONN_E_NODEVICE
        assert not h.value
