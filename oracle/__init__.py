"""oracle -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A CPU fp64 restatement of GoNN's pure-Go attention core (nn/attention.go:107-148
and the tensor ops it calls; the per-function citations are in attn_oracle.c).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only as the checker or the timed CPU baseline. The gonn_amd package
never imports it.

Pinning (each check lives in tests/test_oracle.py):
  attn_fwd          torch fp64 SDPA (library), long-double brute force, golden
                    fixtures, closed forms (Sk=1 -> O=V, Q=0 -> prefix mean,
                    rows sum to 1), the reference's masked-attention invariants
                    (nn/attention_masked_test.go:23-81), the refAttn restatement
                    of benchmark/flashattn/main.go:39-75.
  attn_bwd_autograd torch fp64 autograd, central finite differences with the
                    flashbwd protocol (benchmark/flashbwd/main.go:32-95); with
                    kv_len, torch fp64 autograd through an explicit key mask
                    and exact zeros on the padded keys' dK, dV; with an
                    additive attn_mask, torch fp64 autograd through the same
                    mask in all four of expandAttnMask's shapes.
  attn_bwd_rows     equal to attn_bwd_autograd on every row (1e-12).
  linear / mha_fwd  torch fp64 F.linear / the composed reference sequence.
Planted-mistake tests show each of these checks fails on a plausible bug.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# GONN_ORACLE_LIB selects another build of the same source (the sanitizer
# build of the CPU test suite).
_LIB_PATH = os.environ.get("GONN_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        from . import build as _b  # noqa: F401  (oracle/build.py)
        _b.build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.oracle_attn_fwd.argtypes = [_dp, _dp, _dp, _dp, _dp, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_double, ctypes.c_int, _ip, _ip, ctypes.c_int]
    lib.oracle_attn_bwd_autograd.argtypes = [_dp] * 7 + [ctypes.c_int] * 3 + [
        ctypes.c_double, ctypes.c_int]
    lib.oracle_attn_bwd_autograd_ex.argtypes = [_dp] * 7 + [ctypes.c_int] * 4 + [
        ctypes.c_double, ctypes.c_int, _ip, _dp, ctypes.c_long, ctypes.c_long]
    lib.oracle_attn_bwd_autograd_x.argtypes = [_dp] * 7 + [ctypes.c_int] * 5 + [
        ctypes.c_double, ctypes.c_int, _ip, _dp, ctypes.c_long, ctypes.c_long]
    lib.oracle_attn_fwd_ex.argtypes = [_dp, _dp, _dp, _dp, _dp, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_double, ctypes.c_int, _ip, _dp, ctypes.c_long,
                                       ctypes.c_long, _ip, ctypes.c_int]
    lib.oracle_attn_bwd_rows.argtypes = [_dp] * 9 + [ctypes.c_int] * 3 + [
        ctypes.c_double, ctypes.c_int, _ip, ctypes.c_int, _ip, ctypes.c_int]
    lib.oracle_linear.argtypes = [_dp, _dp, _dp, _dp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.oracle_heads.argtypes = [_dp, _dp] + [ctypes.c_int] * 5
    lib.oracle_attn_fwd_goflow.argtypes = [_dp, _dp, _dp, _dp, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_double, ctypes.c_int]
    lib.oracle_set_mutation.argtypes = [ctypes.c_int]
    lib.oracle_set_threads.argtypes = [ctypes.c_int]
    lib.oracle_get_threads.restype = ctypes.c_int
    _lib = lib
    return lib


def _d(a):
    return a.ctypes.data_as(_dp)


def _c64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


MUTATIONS = {"none": 0, "no_scale": 1, "causal_ge": 2, "transpose_v": 3,
             "no_max_sub": 4, "ds_sign": 5, "lse_log2": 6}


def set_mutation(name: str) -> None:
    """Plant a known mistake in the oracle (mutation tests only)."""
    _load().oracle_set_mutation(MUTATIONS[name])


def set_threads(n: int) -> None:
    _load().oracle_set_threads(int(n))


def get_threads() -> int:
    return int(_load().oracle_get_threads())


def mask_layout(mask, B, H, Sq, Sk):
    """expandAttnMask (nn/attention.go:242-257): an additive mask of shape
    (Sq,Sk), (B*H,Sq,Sk), (B,Sq,Sk) or (B,H,Sq,Sk) as (flat fp64 data, batch
    stride, head stride) in elements; rows are Sk apart."""
    m = _c64(mask)
    s = m.shape
    if s == (Sq, Sk):
        return m.ravel(), 0, 0
    if s == (B * H, Sq, Sk):
        return m.ravel(), H * Sq * Sk, Sq * Sk
    if s == (B, Sq, Sk):
        return m.ravel(), Sq * Sk, 0
    if s == (B, H, Sq, Sk):
        return m.ravel(), H * Sq * Sk, Sq * Sk
    raise ValueError(f"attn mask shape {s} incompatible with (Tq,Tk)=({Sq},{Sk})")


def attn_fwd(Q, K, V, scale=None, causal=False, kv_len=None, H=1, rows=None, attn_mask=None):
    """Forward core. Q (BH,Sq,D), K/V (BH,Sk,D) -> (O (BH,Sq,D), LSE (BH,Sq)).

    kv_len: per-batch valid key counts (length BH/H) or None.
    rows: optional query rows to compute; other rows of O/LSE are NaN.
    attn_mask: optional additive mask in one of mask_layout's shapes.
    """
    lib = _load()
    Q, K, V = _c64(Q), _c64(K), _c64(V)
    BH, Sq, D = Q.shape
    Sk = K.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    O = np.full((BH, Sq, D), np.nan)
    L = np.full((BH, Sq), np.nan)
    kl = None
    if kv_len is not None:
        kl = np.ascontiguousarray(kv_len, dtype=np.int32)
        assert kl.shape[0] * H == BH
    r = None
    nr = 0
    if rows is not None:
        r = np.ascontiguousarray(rows, dtype=np.int32)
        nr = int(r.shape[0])
    am, sb, sh = (None, 0, 0)
    if attn_mask is not None:
        am, sb, sh = mask_layout(attn_mask, BH // H, H, Sq, Sk)
    rc = lib.oracle_attn_fwd_ex(_d(Q), _d(K), _d(V), _d(O), _d(L), BH, H, Sq, Sk, D,
                                float(scale), int(bool(causal)),
                                kl.ctypes.data_as(_ip) if kl is not None else None,
                                _d(am) if am is not None else None, sb, sh,
                                r.ctypes.data_as(_ip) if r is not None else None, nr)
    if rc != 0:
        raise RuntimeError(f"oracle_attn_fwd failed: {rc}")
    return O, L


def attn_bwd_autograd(Q, K, V, dO, scale=None, causal=False, kv_len=None, H=1, attn_mask=None):
    """Backward through the reference's autograd chain -> (dQ, dK, dV).
    kv_len: optional per-batch valid key counts (BH/H entries), the key
    padding mask of ForwardMasked; attn_mask: its additive mask."""
    lib = _load()
    Q, K, V, dO = _c64(Q), _c64(K), _c64(V), _c64(dO)
    BH, S, D = Q.shape
    Sk = K.shape[1]  # != S for cross-attention (top-left causal)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    dQ, dK, dV = np.zeros_like(Q), np.zeros_like(K), np.zeros_like(V)
    kl = None
    if kv_len is not None:
        kl = np.ascontiguousarray(kv_len, dtype=np.int32)
        assert kl.shape == (BH // H,)
    am, sb, sh = (None, 0, 0)
    if attn_mask is not None:
        am, sb, sh = mask_layout(attn_mask, BH // H, H, S, Sk)
    rc = lib.oracle_attn_bwd_autograd_x(_d(Q), _d(K), _d(V), _d(dO), _d(dQ), _d(dK), _d(dV),
                                        BH, int(H), S, Sk, D, float(scale), int(bool(causal)),
                                        kl.ctypes.data_as(_ip) if kl is not None else None,
                                        _d(am) if am is not None else None, sb, sh)
    if rc != 0:
        raise RuntimeError(f"oracle_attn_bwd_autograd failed: {rc}")
    return dQ, dK, dV


def attn_bwd_rows(Q, K, V, O, LSE, dO, scale=None, causal=False, qrows=None, krows=None):
    """Closed-form backward on selected rows (NaN elsewhere) -> (dQ, dK, dV)."""
    lib = _load()
    Q, K, V, O, LSE, dO = (_c64(x) for x in (Q, K, V, O, LSE, dO))
    BH, S, D = Q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    dQ, dK, dV = (np.full_like(Q, np.nan) for _ in range(3))
    qr = np.ascontiguousarray(qrows if qrows is not None else [], dtype=np.int32)
    kr = np.ascontiguousarray(krows if krows is not None else [], dtype=np.int32)
    rc = lib.oracle_attn_bwd_rows(_d(Q), _d(K), _d(V), _d(O), _d(LSE), _d(dO),
                                  _d(dQ), _d(dK), _d(dV), BH, S, D, float(scale),
                                  int(bool(causal)), qr.ctypes.data_as(_ip), int(qr.size),
                                  kr.ctypes.data_as(_ip), int(kr.size))
    if rc != 0:
        raise RuntimeError(f"oracle_attn_bwd_rows failed: {rc}")
    return dQ, dK, dV


def linear(x, W, b=None):
    """Linear.Forward: x (..., in) @ W^T + b."""
    lib = _load()
    x = _c64(x)
    W = _c64(W)
    out_f, in_f = W.shape
    lead = x.shape[:-1]
    N = int(np.prod(lead)) if lead else 1
    y = np.zeros((N, out_f))
    bb = _c64(b) if b is not None else None
    lib.oracle_linear(_d(x), _d(W), _d(bb) if bb is not None else None, _d(y), N, in_f, out_f)
    return y.reshape(*lead, out_f)


def split_heads(x, H):
    """(B,T,E) -> (B*H, T, D), the Reshape+Permute copy of nn/attention.go:120."""
    B, T, E = x.shape
    D = E // H
    out = np.zeros((B, H, T, D))
    _load().oracle_heads(_d(_c64(x)), _d(out), B, T, H, D, 0)
    return out.reshape(B * H, T, D)


def merge_heads(x, B, H):
    """(B*H, T, D) -> (B, T, E), nn/attention.go:146."""
    BH, T, D = x.shape
    out = np.zeros((B, T, H * D))
    _load().oracle_heads(_d(_c64(x)), _d(out), B, T, H, D, 1)
    return out


def mha_fwd(q, k, v, params, H, causal=False, key_pad=None, attn_mask=None):
    """MultiHeadAttention.Forward (nn/attention.go:107-148) / ForwardMasked with
    WithKeyPaddingMask (nn/attention.go:305-341) in fp64.

    params: dict with Wq,bq,Wk,bk,Wv,bv,Wo,bo (Linear weights are (out,in)).
    key_pad: optional (B,Tk) array, nonzero = ignore the key. A suffix mask
    (keys t >= len_b padded) is applied as per-batch key counts; any other is
    added to the scores as keyPaddingMaskAdd's -1e30 (nn/attention.go:
    261-272), after attn_mask, as ForwardMasked orders them (:321-330).
    """
    B, Tq, E = q.shape
    Tk = k.shape[1]
    qp = split_heads(linear(q, params["Wq"], params["bq"]), H)
    kp = split_heads(linear(k, params["Wk"], params["bk"]), H)
    vp = split_heads(linear(v, params["Wv"], params["bv"]), H)
    kv_len = None
    if key_pad is not None:
        kp_arr = np.asarray(key_pad)
        kv_len = []
        for b in range(B):
            nz = np.nonzero(kp_arr[b])[0]
            ln = int(nz[0]) if nz.size else Tk
            kv_len.append(ln)
        if not all(np.all(kp_arr[b, kv_len[b]:] != 0) for b in range(B)):
            kv_len = None
            add = np.where(kp_arr != 0, -1e30, 0.0)
            if attn_mask is None:
                attn_mask = np.broadcast_to(add[:, None, :], (B, Tq, Tk)).copy()
            else:
                _, sb, sh = mask_layout(attn_mask, B, H, Tq, Tk)
                full = np.asarray(attn_mask, dtype=np.float64).reshape(
                    B if sb else 1, H if sh else 1, Tq, Tk)
                attn_mask = np.ascontiguousarray(
                    np.broadcast_to(full, (B, H, Tq, Tk)) + add[:, None, None, :])
    O, _ = attn_fwd(qp, kp, vp, 1.0 / math.sqrt(E // H), causal, kv_len=kv_len, H=H,
                    attn_mask=attn_mask)
    ctx = merge_heads(O, B, H)
    return linear(ctx, params["Wo"], params["bo"])


def ref_attn(Q, K, V, scale, causal):
    """Pure-Python restatement of refAttn (benchmark/flashattn/main.go:39-75):
    two-pass fp64 attention over a materialised row. For small inputs only."""
    Q, K, V = _c64(Q), _c64(K), _c64(V)
    BH, S, d = Q.shape
    O = np.zeros((BH, S, d))
    for bh in range(BH):
        for i in range(S):
            jmax = i + 1 if causal else S
            scores = []
            mx = -math.inf
            for j in range(jmax):
                s = 0.0
                for t in range(d):
                    s += Q[bh, i, t] * K[bh, j, t]
                s *= scale
                scores.append(s)
                if s > mx:
                    mx = s
            tot = 0.0
            for j in range(jmax):
                scores[j] = math.exp(scores[j] - mx)
                tot += scores[j]
            for t in range(d):
                acc = 0.0
                for j in range(jmax):
                    acc += scores[j] * V[bh, j, t]
                O[bh, i, t] = acc / tot
    return O


def attn_fwd_goflow(Q, K, V, scale=None, causal=False):
    """GoNN's CPU forward core with GoNN's pass structure (every op a whole-
    tensor pass into a new buffer, broadcasts materialised, elementwise loops
    on one thread, GEMMs threaded): the timed CPU baseline. Q, K, V (BH,S,D)
    -> O (BH,S,D), equal to attn_fwd's O. Needs ~6 fp64 copies of the
    (BH,S,S) scores in memory."""
    Q, K, V = _c64(Q), _c64(K), _c64(V)
    BH, S, D = Q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    O = np.empty_like(Q)
    rc = _load().oracle_attn_fwd_goflow(_d(Q), _d(K), _d(V), _d(O), BH, S, D, float(scale),
                                        int(bool(causal)))
    if rc:
        raise MemoryError(f"oracle_attn_fwd_goflow: {rc}")
    return O
