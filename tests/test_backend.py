"""The backend contract around the attention core (backend/backend.go:61-78):
the CPU backend's row-major batched GEMM against a naive triple loop at
1e-12 (the reference's own bar, backend/backend_test.go:47-86), backend
selection (Use / Current), and the device GEMM entry point's argument and
no-device paths (no CPU fallback)."""
import ctypes

import numpy as np
import pytest

from gonn_amd import _lib, backend, hip
from gonn_amd._lib import GONN_E_INVALID, GONN_E_NODEVICE


def _naive(A, B, batch, m, k, n, ta, tb):
    A = A.reshape(batch, *((k, m) if ta else (m, k)))
    B = B.reshape(batch, *((n, k) if tb else (k, n)))
    C = np.zeros((batch, m, n))
    for z in range(batch):
        for i in range(m):
            for j in range(n):
                s = 0.0
                for p in range(k):
                    a = A[z, p, i] if ta else A[z, i, p]
                    b = B[z, j, p] if tb else B[z, p, j]
                    s += a * b
                C[z, i, j] = s
    return C.reshape(-1)


# The case list of backend/backend_test.go:54-66: plain 2D in every
# transpose combination, batched, degenerate 1x1x1.
_CASES = [(1, 3, 4, 5, False, False), (1, 3, 4, 5, True, False), (1, 3, 4, 5, False, True),
          (1, 3, 4, 5, True, True), (4, 2, 3, 2, False, False), (4, 2, 3, 2, True, True),
          (2, 1, 1, 1, False, False), (3, 5, 2, 4, False, True), (3, 5, 7, 4, True, False)]


@pytest.mark.parametrize("case", _CASES, ids=lambda c: "-".join(map(str, c)))
def test_cpu_backend_gemm_matches_naive(case):
    batch, m, k, n, ta, tb = case
    rng = np.random.default_rng(7)
    A = rng.standard_normal(batch * m * k)
    B = rng.standard_normal(batch * k * n)
    be = backend.NewCPU()
    assert be.Name() == "cpu"
    got = be.Gemm(A, B, batch, m, k, n, ta, tb)
    ref = _naive(A, B, batch, m, k, n, ta, tb)
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) <= 1e-12


def test_cpu_backend_empty_batch():
    # backend_test.go:82-85: batch 0 gives an empty result.
    assert backend.NewCPU().Gemm(np.zeros(0), np.zeros(0), 0, 3, 4, 5).size == 0


def test_use_current_concurrent():
    # backend_test.go:90-111: Use/Current from many threads, restored after.
    import threading
    start = backend.Current()
    errs = []

    def worker():
        for _ in range(1000):
            prev = backend.Use(backend.CPUBackend())
            if backend.Current() is None:
                errs.append("nil")
                return
            backend.Use(prev)

    ts = [threading.Thread(target=worker) for _ in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    backend.Use(start)
    assert not errs and backend.Current().Name() == "cpu"


def test_use_returns_previous_and_linear_dispatches():
    calls = []

    class Spy(backend.CPUBackend):
        def Gemm(self, *a, **kw):
            calls.append(a[2:6])
            return super().Gemm(*a, **kw)

    prev = backend.Use(Spy())
    try:
        from gonn_amd import nn
        lin = nn.Linear(np.ones((3, 4)), np.zeros(3))
        y = lin.forward(np.ones((2, 5, 4)))
        assert y.shape == (2, 5, 3) and np.all(y == 4.0)
        assert calls == [(1, 10, 4, 3)]
    finally:
        backend.Use(prev)
    assert backend.Current() is prev


def test_gemm_entry_checks():
    lib = _lib.load()
    dp = ctypes.POINTER(ctypes.c_double)
    x = np.zeros(16)
    p = x.ctypes.data_as(dp)
    assert lib.gonn_hip_gemm_f64(p, p, p, -1, 2, 2, 2, 0, 0) == GONN_E_INVALID
    assert lib.gonn_hip_gemm_f64(None, p, p, 1, 2, 2, 2, 0, 0) == GONN_E_INVALID
    assert lib.gonn_hip_gemm_f64(p, p, p, 0, 2, 2, 2, 0, 0) == 0  # empty result
    if not hip.Available():
        assert lib.gonn_hip_gemm_f64(p, p, p, 1, 2, 2, 2, 0, 0) == GONN_E_NODEVICE
        with pytest.raises(RuntimeError):
            backend.HIPBackend()


def test_kind_values_are_the_abi():
    # backend/backend.go:26-58 and gonn_cuda.h:13-28: append-only values.
    import re
    from gonn_amd import _lib
    hdr = open(__file__.rsplit("/tests/", 1)[0] + "/include/gonn_hip.h").read()
    for name, val in re.findall(r"GONN_(UN_\w+|BIN_\w+) = (\d+)", hdr):
        assert getattr(_lib, "GONN_" + name) == int(val)
    assert (backend.UnaryReLU, backend.UnaryLog, backend.UnaryGELUExact) == (0, 4, 7)
    assert (backend.BinaryAdd, backend.BinaryDiv) == (0, 3)


def test_cpu_backend_is_not_an_elementwiser():
    # backend_test.go:117-126: the CPU backend must not implement it.
    cpu = backend.NewCPU()
    assert not hasattr(cpu, "Unary") and not hasattr(cpu, "Binary")
    x = np.ones(1 << 17)
    out = np.zeros_like(x)
    prevp = backend.GetDispatchPolicy()
    backend.SetDispatchPolicy(backend.DispatchPolicy(0, 0))
    try:
        assert not backend.dispatch_unary(backend.UnaryExp, x, out)
        assert not backend.dispatch_binary(backend.BinaryAdd, x, x, out)
    finally:
        backend.SetDispatchPolicy(prevp)
    assert not out.any()


def test_dispatch_policy_thresholds():
    # tensor/dispatch.go:60-109: defaults, UnaryNone never dispatches.
    calls = []

    class Spy(backend.CPUBackend):
        def Unary(self, kind, a, out):
            calls.append(("u", kind, np.size(a)))
            return True

        def Binary(self, kind, a, b, out):
            calls.append(("b", kind, np.size(a)))
            return True

    p = backend.GetDispatchPolicy()
    assert p.UnaryMinElems == 1 << 16 and p.BinaryMinElems >= 2 ** 62
    prev = backend.Use(Spy())
    try:
        small, big = np.zeros((1 << 16) - 1), np.zeros(1 << 16)
        assert not backend.dispatch_unary(backend.UnaryTanh, small, small)
        assert backend.dispatch_unary(backend.UnaryTanh, big, big)
        assert not backend.dispatch_unary(backend.UnaryNone, big, big)
        assert not backend.dispatch_binary(backend.BinaryMul, big, big, big)
    finally:
        backend.Use(prev)
    assert calls == [("u", backend.UnaryTanh, 1 << 16)]


def test_elementwise_entry_checks():
    lib = _lib.load()
    dp = ctypes.POINTER(ctypes.c_double)
    x = np.zeros(8)
    p = x.ctypes.data_as(dp)
    assert lib.gonn_hip_unary_f64(8, p, p, 8) == GONN_E_INVALID
    assert lib.gonn_hip_unary_f64(-1, p, p, 8) == GONN_E_INVALID
    assert lib.gonn_hip_binary_f64(4, p, p, p, 8) == GONN_E_INVALID
    assert lib.gonn_hip_unary_f64(0, p, p, -1) == GONN_E_INVALID
    assert lib.gonn_hip_unary_f64(0, None, None, 0) == 0
    assert lib.gonn_hip_binary_f64(0, None, p, p, 8) == GONN_E_INVALID
    b = _lib.Buf(0, 0, _lib.GONN_F32)
    assert lib.gonn_hip_unary_f64_dev(0, ctypes.byref(b), ctypes.byref(b), 4, None) == GONN_E_INVALID
    if not hip.Available():
        assert lib.gonn_hip_unary_f64(0, p, p, 8) == GONN_E_NODEVICE
        assert lib.gonn_hip_binary_f64(0, p, p, p, 8) == GONN_E_NODEVICE


def test_mask_strides_follow_expand_attn_mask():
    # nn/attention.go:242-257: the four accepted shapes and the panic otherwise.
    B, H, Sq, Sk = 2, 3, 5, 7
    assert hip.mask_strides((Sq, Sk), B, H, Sq, Sk) == (0, 0)
    assert hip.mask_strides((B, Sq, Sk), B, H, Sq, Sk) == (Sq * Sk, 0)
    assert hip.mask_strides((B * H, Sq, Sk), B, H, Sq, Sk) == (H * Sq * Sk, Sq * Sk)
    assert hip.mask_strides((B, H, Sq, Sk), B, H, Sq, Sk) == (H * Sq * Sk, Sq * Sk)
    for bad in ((Sk, Sq), (B, Sq, Sk + 1), (B * H + 1, Sq, Sk), (1, B, H, Sq, Sk)):
        with pytest.raises(ValueError, match="attn mask shape"):
            hip.mask_strides(bad, B, H, Sq, Sk)


def test_key_padding_mask_to_kv_len():
    # keyPaddingMaskAdd (nn/attention.go:261-272): nonzero = ignore; suffix
    # masks that leave a key become per-sequence key counts.
    from gonn_amd import nn
    m = np.zeros((4, 6))
    m[1, 4:] = 1
    m[3, 5] = 2.5        # any nonzero value pads
    assert list(nn._kv_len_from_mask(m, 4, 6)) == [6, 4, 6, 5]
    assert nn._kv_len_from_mask(None, 4, 6) is None
    holes = m.copy()
    holes[0, 2] = 1      # a padded key before valid ones
    with pytest.raises(ValueError, match="suffix"):
        nn._kv_len_from_mask(holes, 4, 6)
    full = m.copy()
    full[2, :] = 1       # every key padded: GoNN's uniform average, not defined here
    with pytest.raises(ValueError, match="no unblocked key"):
        nn._kv_len_from_mask(full, 4, 6)
    with pytest.raises(ValueError, match="key padding mask shape"):
        nn._kv_len_from_mask(np.zeros((4, 5)), 4, 6)


def test_core_masks_forms():
    """ForwardMasked's masks as the fused core takes them (nn._core_masks):
    suffix padding -> kv_len; holes -> keyPaddingMaskAdd's -1e30 added to the
    additive mask; rows shifted by their in-window maximum. Checked against a
    direct restatement on small cases, and by softmax invariance: the shifted
    mask gives the same probabilities as GoNN's scores + mask in fp64."""
    from gonn_amd import nn
    B, H, Tq, Tk = 2, 3, 5, 7
    r = np.random.default_rng(3)
    pad = np.zeros((B, Tk))
    pad[1, 5:] = 1
    kv, am, c = nn._core_masks(pad, None, B, H, Tq, Tk, False)
    assert list(kv) == [7, 5] and am is None and c is False
    # a zero-max mask passes through unchanged (no copy)
    z = np.zeros((Tq, Tk))
    z[:, 3] = -1e30
    kv, am, c = nn._core_masks(None, z, B, H, Tq, Tk, True)
    assert kv is None and am is z and c is True
    # holes + a (B*H, Tq, Tk) mask with a large common offset, causal
    holes = pad.copy()
    holes[0, 2] = 1
    um = r.standard_normal((B * H, Tq, Tk)) - 1e4
    scores = r.standard_normal((B, H, Tq, Tk))
    kv, am, c = nn._core_masks(holes, um, B, H, Tq, Tk, True)
    assert kv is None and am.shape == (B, H, Tq, Tk) and c is True
    win = np.arange(Tk)[None, :] <= np.arange(Tq)[:, None]

    def softmax(x):
        x = np.where(win, x, -np.inf)
        e = np.exp(x - x.max(-1, keepdims=True))
        return e / e.sum(-1, keepdims=True)
    ref = softmax(scores + um.reshape(B, H, Tq, Tk) + np.where(holes != 0, -1e30, 0.0)[:, None, None])
    # (GoNN forms scores - 1e4 in fp64: its own rounding is ~1e-12 of the exponent)
    np.testing.assert_allclose(softmax(scores + am), ref, rtol=1e-9, atol=1e-300)
    inwin = np.where(win, am, -np.inf).max(-1)
    assert np.all(inwin == 0.0)
    # suffix padding + a (Tq, Tk) mask: the window max depends on kv_len
    tm = r.standard_normal((Tq, Tk)) * 3
    kv, am, c = nn._core_masks(pad, tm, B, H, Tq, Tk, False)
    assert list(kv) == [7, 5] and am.shape == (B, Tq, Tk)
    np.testing.assert_array_equal(am[0], tm - tm.max(-1, keepdims=True))
    np.testing.assert_array_equal(am[1], tm - tm[:, :5].max(-1, keepdims=True))
    b0 = np.zeros((Tq, Tk))
    b0[0, 0] = -1e30
    kv, am, c = nn._core_masks(None, b0, B, H, Tq, Tk, False)  # non-causal: keys 1.. remain
    assert am is b0 and c is False
    with pytest.raises(ValueError, match="attn mask shape"):
        nn._core_masks(None, np.zeros((Tq, Tk + 1)), B, H, Tq, Tk, False)


def test_core_masks_blocked_rows():
    """Rows with no unblocked key (nn._core_masks' whole-row form): GoNN adds
    causalMaskAdd, the attn mask and keyPaddingMaskAdd as fp64 -1e30 terms
    (nn/attention.go:185-196, :261-272, :321-330), which absorb the scores,
    so a blocked row is a uniform average over the keys whose summed mask is
    the row's maximum, future keys included. The whole-row form must give
    GoNN's probabilities (scores + its masks in fp64, max-subtracted softmax)
    for every row, in the reference's order of additions; rows it cannot
    reproduce are refused."""
    from gonn_amd import nn
    B, H, Tq, Tk = 2, 2, 6, 6
    r = np.random.default_rng(4)
    scores = r.standard_normal((B, H, Tq, Tk)) * 3

    def gonn_probs(causal, attn, keypad):
        x = scores.copy()
        if causal:
            x = x + np.where(np.arange(Tk)[None, :] > np.arange(Tq)[:, None], -1e30, 0.0)
        if attn is not None:
            x = x + np.broadcast_to(attn, x.shape) if attn.ndim == 2 else \
                x + attn.reshape(B, -1, Tq, Tk)
        if keypad is not None:
            x = x + np.where(keypad != 0, -1e30, 0.0)[:, None, None, :]
        e = np.exp(x - x.max(-1, keepdims=True))
        return e / e.sum(-1, keepdims=True)

    def probs(am):
        x = scores + (am[:, None] if am.ndim == 3 else am)
        e = np.exp(x - x.max(-1, keepdims=True))
        return e / e.sum(-1, keepdims=True)

    cases = []
    # a fully padded sequence (suffix form with no key left), non-causal
    full = np.zeros((B, Tk))
    full[0] = 1
    full[1, 4:] = 1
    cases.append((False, None, full))
    # causal with padded leading keys: rows 0-1 keep none of theirs; their
    # maximum class holds the padded keys up to the row and the unpadded
    # future keys (each one -1e30), not the padded future keys (-2e30)
    lead = np.zeros((B, Tk))
    lead[:, :2] = 1
    cases.append((True, None, lead))
    # causal, an attn mask blocking row 0's only key, plus holes
    b0 = r.standard_normal((Tq, Tk))
    b0[0, 0] = -1e30
    holes = np.zeros((B, Tk))
    holes[1, 3] = 1
    cases.append((True, b0, holes))
    for causal, attn, keypad in cases:
        kv, am, c = nn._core_masks(keypad, attn, B, H, Tq, Tk, causal)
        assert kv is None and c is False
        ref = gonn_probs(causal, attn, keypad)
        np.testing.assert_allclose(probs(am), ref, rtol=1e-12, atol=1e-300)
    # the second case's row 0 of batch 0: padded key 0 and unpadded keys 2..5
    ref = gonn_probs(True, None, lead)[0, 0, 0]
    np.testing.assert_allclose(ref, [0.2, 0, 0.2, 0.2, 0.2, 0.2], atol=1e-15)
    # refused: a blocked row whose best value keeps part of the score in fp64
    mid = np.zeros((Tq, Tk))
    mid[0] = -1e20
    with pytest.raises(ValueError, match="between"):
        nn._core_masks(None, mid, B, H, Tq, Tk, False)
    # refused: a row of -inf (NaN in the reference)
    ninf = np.zeros((Tq, Tk))
    ninf[2] = -np.inf
    with pytest.raises(ValueError, match="between"):
        nn._core_masks(None, ninf, B, H, Tq, Tk, False)


def test_resident_layer_and_cache_need_a_device():
    # No CPU fallback: without a gfx950 device the device-resident objects
    # refuse to construct (gonn_hip_*_create returns GONN_E_NODEVICE).
    from gonn_amd import nn
    if hip.Available():
        pytest.skip("a device is present")
    E = 64
    w = np.eye(E)
    mha = nn.MultiHeadAttention(E, 4, w, None, w, None, w, None, w, None)
    with pytest.raises(Exception):
        mha.to_device()
    with pytest.raises(hip.GonnHipError):
        hip.DeviceMHA(E, 4, w, None, w, None, w, None, w, None)
    with pytest.raises(hip.GonnHipError):
        hip.KVCache(1, 1, 16, 64)
