"""Seeded randomized parity sweep of the fused core through the device API:
shapes, modes and options drawn together (ragged Sq and Sk, cross-attention,
causal, key padding with empty sequences, additive masks in each of
expandAttnMask's shapes, D in {64, 128}), forward and backward against the
oracle. Each case prints its parameters before it runs. Sizes stay small so
the oracle's materialised chain finishes in well under a second per case."""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

N_CASES = 24


def _case(i):
    r = np.random.default_rng(5000 + i)
    B, H = int(r.integers(1, 4)), int(r.integers(1, 4))
    D = int(r.choice([64, 128]))
    Sq = int(r.integers(1, 260))
    Sk = Sq if r.random() < 0.5 else int(r.integers(1, 260))
    causal = bool(r.random() < 0.5)
    mode = str(r.choice(["fp32", "bf16"]))
    kv = None
    if r.random() < 0.5:
        kv = r.integers(0, Sk + 1, size=B).astype(np.int32)
        kv[0] = Sk  # at least one full sequence
    mkind = None if r.random() < 0.5 else str(r.choice(["TqTk", "BTqTk", "BHTqTk3", "BHTqTk4"]))
    return dict(B=B, H=H, D=D, Sq=Sq, Sk=Sk, causal=causal, mode=mode, kv=kv, mkind=mkind,
                seed=6000 + i)


def _mask(kind, B, H, Sq, Sk, r):
    shape = {"TqTk": (Sq, Sk), "BTqTk": (B, Sq, Sk), "BHTqTk3": (B * H, Sq, Sk),
             "BHTqTk4": (B, H, Sq, Sk)}[kind]
    m = r.standard_normal(shape)
    # Block key 1 on some rows. Key 0 stays open: a row whose every key
    # carries -1e30 has no finite log-sum-exp in fp32 (outside the definition).
    if Sk >= 2:
        m[..., 1] = np.where(r.random(shape[:-1]) < 0.3, -1e30, m[..., 1])
    return m


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_case(i):
    from gonn_amd import hip
    c = _case(i)
    B, H, D, Sq, Sk = c["B"], c["H"], c["D"], c["Sq"], c["Sk"]
    say(f"[random {i}] B={B} H={H} D={D} Sq={Sq} Sk={Sk} causal={c['causal']} "
        f"mode={c['mode']} kv={None if c['kv'] is None else list(c['kv'])} mask={c['mkind']}")
    r = np.random.default_rng(c["seed"])
    q, g = (r.standard_normal((B * H, Sq, D)) for _ in range(2))
    k, v = (r.standard_normal((B * H, Sk, D)) for _ in range(2))
    m = _mask(c["mkind"], B, H, Sq, Sk, r) if c["mkind"] else None
    dev = lambda x, S: torch.from_numpy(x.astype(np.float32)).cuda().reshape(B, H, S, D)  # noqa: E731
    dq_, dk_, dv_, dg_ = dev(q, Sq), dev(k, Sk), dev(v, Sk), dev(g, Sq)
    kl = torch.from_numpy(c["kv"]).cuda() if c["kv"] is not None else None
    md = torch.from_numpy(m.astype(np.float32)).cuda() if m is not None else None
    o, l = hip.attn_fwd(dq_, dk_, dv_, causal=c["causal"], mode=c["mode"], kv_len=kl, attn_mask=md)
    dq, dk, dv = hip.attn_bwd(dq_, dk_, dv_, o, l, dg_, causal=c["causal"], mode=c["mode"],
                              kv_len=kl, attn_mask=md)
    torch.cuda.synchronize()
    sc = 1.0 / math.sqrt(D)
    ro, rl = oracle.attn_fwd(q, k, v, sc, c["causal"], kv_len=c["kv"], H=H, attn_mask=m)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, sc, c["causal"], kv_len=c["kv"], H=H,
                                          attn_mask=m)
    # Every call runs in the stated mode: that mode's bar.
    fmode = c["mode"]
    live = np.ones(B * H, bool) if c["kv"] is None else np.repeat(c["kv"] > 0, H)
    o = o.reshape(B * H, Sq, D).cpu().numpy()
    assert_close(o[live], ro[live], fmode, f"O case {i}")
    assert_close(l.cpu().numpy()[live], rl[live], fmode, f"LSE case {i}")
    for got, ref, S, n in ((dq, rq, Sq, "dQ"), (dk, rk, Sk, "dK"), (dv, rv, Sk, "dV")):
        got = got.reshape(B * H, S, D).cpu().numpy()
        assert_close(got[live], ref[live], fmode, f"{n} case {i}")
        assert np.all(got[~live] == 0.0), f"{n} case {i}: a sequence with no key"
    assert np.all(o[~live] == 0.0)


def test_concurrent_calls_on_separate_streams():
    """The entry points are reentrant (gonn_hip.h): threads running forward +
    backward on their own streams at once give exactly what each call gives
    alone (the reference's contract allows concurrent Backward calls,
    tensor/autograd.go:10-32)."""
    import threading
    from gonn_amd import hip
    cases = []
    for t in range(4):
        r = np.random.default_rng(7000 + t)
        B, H, S, D = 2, 2, 96 + 37 * t, (64, 128)[t % 2]
        mode = ("fp32", "bf16")[t // 2]
        x = [torch.from_numpy(r.standard_normal((B, H, S, D)).astype(np.float32)).cuda()
             for _ in range(4)]
        cases.append((x, mode))
    torch.cuda.synchronize()

    def run(x, mode):
        o, l = hip.attn_fwd(x[0], x[1], x[2], causal=True, mode=mode)
        g = hip.attn_bwd(x[0], x[1], x[2], o, l, x[3], causal=True, mode=mode)
        return [o, l, *g]

    ref = [run(*c) for c in cases]
    torch.cuda.synchronize()
    got = [None] * len(cases)
    errs = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(3):
                    got[i] = run(*cases[i])
            s.synchronize()
        except Exception as e:  # surfaced below
            errs.append(repr(e))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    torch.cuda.synchronize()
    assert not errs, errs
    for i in range(len(cases)):
        for a, b in zip(got[i], ref[i]):
            assert torch.equal(a, b), f"thread {i}"
