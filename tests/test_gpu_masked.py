"""GPU parity of the wider fused gate: cross-attention (Sq != Sk, top-left
causal mask) and ForwardMasked's prefix key padding on the fused forward.

Reference semantics: causalMaskAdd (nn/attention.go:185-196) and
keyPaddingMaskAdd (:261-272) both add -1e30, which gives masked keys an
exactly-zero weight in fp64; ForwardMasked adds both (:321-330). The oracle
restates that (attn_oracle.c), so the GPU output is compared with it at the
bar of the arithmetic mode (fp32-MFMA max-abs 1e-4; bf16-MFMA 2e-2 + 1e-2|ref|).
A sequence with no valid key is defined here as O = 0, LSE = -inf.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_fwd_kv_len_and_cross_shapes(mode, D, causal):
    from gonn_amd import hip
    B, H, Sq, Sk = 3, 2, 70, 150
    lens = np.array([150, 37, 0], dtype=np.int32)
    say(f"[masked] fwd mode={mode} D={D} causal={causal} Sq={Sq} Sk={Sk} lens={list(lens)}")
    q = randn((B * H, Sq, D), 800 + D)
    k = randn((B * H, Sk, D), 801 + D)
    v = randn((B * H, Sk, D), 802 + D)
    dev = [torch.from_numpy(x).cuda().reshape(B, H, -1, D) for x in (q, k, v)]
    kl = torch.from_numpy(lens).cuda()
    o, l = hip.attn_fwd(*dev, causal=causal, mode=mode, kv_len=kl)
    torch.cuda.synchronize()
    o = o.reshape(B * H, Sq, D).cpu().numpy()
    l = l.cpu().numpy()
    ro, rl = oracle.attn_fwd(q, k, v, 1.0 / math.sqrt(D), causal, kv_len=lens, H=H)
    live = np.repeat(lens > 0, H)
    assert_close(o[live], ro[live], mode, f"O kv_len {mode} D={D} causal={causal}")
    assert_close(l[live], rl[live], mode, f"LSE kv_len {mode} D={D} causal={causal}")
    assert np.all(o[~live] == 0.0) and np.all(np.isneginf(l[~live]))


def test_fwd_kv_len_clamped_and_absent_equal_full():
    """kv_len >= Sk for every sequence is the same as no kv_len (bit-identical)."""
    from gonn_amd import hip
    B, H, S, D = 2, 4, 200, 128
    dev = [torch.from_numpy(randn((B, H, S, D), 810 + i)).cuda() for i in range(3)]
    o0, l0 = hip.attn_fwd(*dev, causal=True, mode="bf16")
    kl = torch.tensor([S, S + 1000], dtype=torch.int32, device="cuda")
    o1, l1 = hip.attn_fwd(*dev, causal=True, mode="bf16", kv_len=kl)
    torch.cuda.synchronize()
    assert torch.equal(o0, o1) and torch.equal(l0, l1)


@pytest.mark.parametrize("d", [64, 100, 128])
def test_f64_ex_entry(d):
    from gonn_amd import hip
    B, H, Sq, Sk = 2, 3, 33, 90
    lens = np.array([90, 12], dtype=np.int32)
    say(f"[masked] FlashAttnF64Ex d={d}")
    q = randn((B * H, Sq, d), 820 + d).astype(np.float64)
    k = randn((B * H, Sk, d), 821 + d).astype(np.float64)
    v = randn((B * H, Sk, d), 822 + d).astype(np.float64)
    for causal in (False, True):
        O, L = hip.FlashAttnF64Ex(q, k, v, B, H, Sq, Sk, d, 1.0 / math.sqrt(d), causal,
                                  kv_len=lens, lse=True)
        ro, rl = oracle.attn_fwd(q, k, v, 1.0 / math.sqrt(d), causal, kv_len=lens, H=H)
        assert_close(O.reshape(ro.shape), ro, "fp32", f"FlashAttnF64Ex d={d} causal={causal}")
        assert_close(L.reshape(rl.shape), rl, "fp32", f"FlashAttnF64Ex LSE d={d} causal={causal}")


def _params(E, seed):
    s = 1.0 / math.sqrt(E)
    p = {}
    for i, n in enumerate(("q", "k", "v", "o")):
        p["W" + n] = randn((E, E), seed + 2 * i).astype(np.float64) * s
        p["b" + n] = randn((E,), seed + 2 * i + 1).astype(np.float64) * 0.1
    return p


@pytest.mark.parametrize("causal", [False, True])
def test_mha_forward_masked_and_cross_attention(causal):
    from gonn_amd import nn
    E, H, B, Tq, Tk = 256, 4, 3, 40, 64
    say(f"[masked] MHA forward_masked / cross causal={causal}")
    p = _params(E, 840)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    x = randn((B, Tk, E), 850).astype(np.float64)
    mem = randn((B, Tk, E), 851).astype(np.float64)
    q = randn((B, Tq, E), 852).astype(np.float64)
    pad = np.zeros((B, Tk))
    pad[1, 50:] = 1
    pad[2, 7:] = 1
    # self-attention with key padding (Tq == Tk)
    got = mha.forward_masked(x, x, x, causal=causal, key_padding_mask=pad)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=causal, key_pad=pad)
    assert_close(got, ref, "fp32", f"forward_masked causal={causal}")
    # cross-attention (Tq != Tk), with and without padding
    got = mha.forward_fused(q, mem, mem, causal)
    ref = oracle.mha_fwd(q, mem, mem, p, H, causal=causal)
    assert_close(got, ref, "fp32", f"cross-attention causal={causal}")
    got = mha.forward_masked(q, mem, mem, causal=causal, key_padding_mask=pad)
    ref = oracle.mha_fwd(q, mem, mem, p, H, causal=causal, key_pad=pad)
    assert_close(got, ref, "fp32", f"cross-attention + padding causal={causal}")
    # a padding mask with holes (added as -1e30), with a padded leading key
    # on a row that keeps later keys
    holes = pad.copy()
    holes[0, 3] = 1
    holes[2, 1 if causal else 0] = 1
    got = mha.forward_masked(x, x, x, causal=causal, key_padding_mask=holes)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=causal, key_pad=holes)
    assert_close(got, ref, "fp32", f"forward_masked holes causal={causal}")
    # rows with no unblocked key: GoNN's -1e30 terms absorb their scores,
    # so each is a uniform average over the keys whose summed mask is the
    # row's maximum (future keys included, with their causal -1e30); the
    # mirror runs them in the whole-row form. A sequence with every key
    # padded; padded leading keys (under causal, the first rows keep none of
    # their own); an attn mask blocking row 0's only key.
    full = pad.copy()
    full[1] = 1
    got = mha.forward_masked(x, x, x, causal=causal, key_padding_mask=full)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=causal, key_pad=full)
    assert_close(got, ref, "fp32", f"forward_masked fully padded causal={causal}")
    lead = np.zeros((B, Tk))
    lead[:, :3] = 1
    lead[2, 60:] = 1
    got = mha.forward_masked(x, x, x, causal=causal, key_padding_mask=lead)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=causal, key_pad=lead)
    assert_close(got, ref, "fp32", f"forward_masked padded leading keys causal={causal}")
    am = randn((Tk, Tk), 853).astype(np.float64)
    am[0, 0] = -1e30
    am[5, :] = -1e30
    got = mha.forward_masked(x, x, x, causal=causal, attn_mask=am, key_padding_mask=pad)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=causal, key_pad=pad, attn_mask=am)
    assert_close(got, ref, "fp32", f"forward_masked blocked rows + attn mask causal={causal}")
    # refused: a blocked row whose best value keeps part of the score in fp64
    mid = np.zeros((Tk, Tk))
    mid[4, :] = -1e20
    with pytest.raises(ValueError, match="between"):
        mha.forward_masked(x, x, x, causal=causal, attn_mask=mid)
    with pytest.raises(ValueError):
        mha.forward_masked(x, x, x, dropout=0.1)
    with pytest.raises(ValueError):
        mha.forward_masked(x, x, x, attn_mask=np.zeros((Tk, Tk + 1)))


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_bwd_kv_len_matches_oracle_autograd(mode, D, causal):
    """Backward of ForwardMasked's key padding (kv_len) against GoNN's autograd
    chain through the same additive masks (oracle.attn_bwd_autograd with
    kv_len, pinned to torch fp64 autograd): padded keys get dK = dV = 0
    exactly, a sequence with no key gets all-zero gradients."""
    from gonn_amd import hip
    B, H, S = 4, 2, 150
    lens = np.array([150, 37, 0, 129], dtype=np.int32)
    say(f"[masked] bwd mode={mode} D={D} causal={causal} S={S} lens={list(lens)}")
    q, k, v, g = (randn((B * H, S, D), 820 + D + i) for i in range(4))
    dev = [torch.from_numpy(x).cuda().reshape(B, H, S, D) for x in (q, k, v, g)]
    kl = torch.from_numpy(lens).cuda()
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode=mode, kv_len=kl)
    dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode=mode, kv_len=kl)
    torch.cuda.synchronize()
    dq, dk, dv = (t.reshape(B * H, S, D).cpu().numpy() for t in (dq, dk, dv))
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H)
    live = np.repeat(lens > 0, H)
    assert_close(dq[live], rq[live], mode, f"dQ kv_len {mode} D={D} causal={causal}")
    assert_close(dk[live], rk[live], mode, f"dK kv_len {mode} D={D} causal={causal}")
    assert_close(dv[live], rv[live], mode, f"dV kv_len {mode} D={D} causal={causal}")
    for bh in range(B * H):
        n = lens[bh // H]
        assert np.all(dk[bh, n:] == 0.0) and np.all(dv[bh, n:] == 0.0), bh
        if n == 0:
            assert np.all(dq[bh] == 0.0)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_bwd_kv_len_full_equals_absent(mode):
    """kv_len >= S for every sequence gives the same gradients as no kv_len,
    bit for bit."""
    from gonn_amd import hip
    B, H, S, D = 2, 2, 200, 128
    dev = [torch.from_numpy(randn((B, H, S, D), 840 + i)).cuda() for i in range(4)]
    o, l = hip.attn_fwd(*dev[:3], causal=True, mode=mode)
    g0 = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=True, mode=mode)
    kl = torch.tensor([S, S + 5], dtype=torch.int32, device="cuda")
    g1 = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=True, mode=mode, kv_len=kl)
    torch.cuda.synchronize()
    for a, b in zip(g0, g1):
        assert torch.equal(a, b)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_fused_attn_diff_with_key_padding(mode):
    """nn.fused_attn_diff with kv_len: the fp64 entry points
    (gonn_hip_flash_attn_f64_ex / _bwd_ex) give the forward and the node's
    backward of ForwardMasked's key padding; against the oracle's forward and
    autograd chain."""
    from gonn_amd import hip, nn
    prev = hip.AttnMode()
    hip.SetAttnMode(mode)
    try:
        B, H, S, D = 3, 2, 90, 64
        lens = np.array([90, 41, 7], dtype=np.int32)
        q, k, v, g = (randn((B * H, S, D), 860 + i) for i in range(4))
        O, node = nn.fused_attn_diff(q, k, v, B * H, S, D, 1 / math.sqrt(D), True,
                                     kv_len=lens, H=H)
        dq, dk, dv = (x.reshape(B * H, S, D) for x in node(g.ravel()))
    finally:
        hip.SetAttnMode(prev)
    ro, _ = oracle.attn_fwd(q, k, v, 1 / math.sqrt(D), True, kv_len=lens, H=H)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=True, kv_len=lens, H=H)
    assert_close(O.reshape(B * H, S, D), ro, mode, f"fused_attn_diff O {mode}")
    assert_close(dq, rq, mode, f"fused_attn_diff dQ {mode}")
    assert_close(dk, rk, mode, f"fused_attn_diff dK {mode}")
    assert_close(dv, rv, mode, f"fused_attn_diff dV {mode}")
    for bh in range(B * H):
        assert np.all(dk[bh, lens[bh // H]:] == 0.0)


def _mask_of(kind, B, H, Sq, Sk, seed):
    """An additive mask in one of expandAttnMask's shapes, with a blocked
    (-1e30) key column and a band of blocked scores, plus its dense
    (B*H, Sq, Sk) expansion."""
    rng = np.random.default_rng(seed)
    full = rng.standard_normal((B, H, Sq, Sk)) * 1.5
    full[..., 3] = -1e30
    for i in range(Sq):
        full[:, :, i, max(0, i - 40):max(0, i - 30)] = -1e30  # a blocked band
    if kind == "TqTk":
        full[:] = full[0, 0]
        m = full[0, 0]
    elif kind == "BTqTk":
        full[:] = full[:, :1]
        m = full[:, 0]
    elif kind == "BHTqTk3":
        m = full.reshape(B * H, Sq, Sk)
    else:
        m = full
    return np.ascontiguousarray(m), full.reshape(B * H, Sq, Sk)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("kind", ["TqTk", "BTqTk", "BHTqTk3", "BHTqTk4"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_attn_mask_fwd_bwd_matches_oracle(mode, kind, causal, D):
    """WithAttnMask on the fused path (device API): forward and backward
    against the oracle's reference chain with the same additive mask, key
    padding and causal mask. The forward runs the stated mode's kernels (the
    bf16 ones add the mask in log2 units to each completed S^T tile), and so
    does the backward; everything is held to the stated mode's bar."""
    from gonn_amd import hip
    B, H, S = 2, 2, 100
    lens = np.array([100, 71], dtype=np.int32)
    say(f"[masked] attn_mask {kind} mode={mode} causal={causal}")
    m, _ = _mask_of(kind, B, H, S, S, 870)
    q, k, v, g = (randn((B * H, S, D), 880 + i) for i in range(4))
    dev = [torch.from_numpy(x).cuda().reshape(B, H, S, D) for x in (q, k, v, g)]
    kl = torch.from_numpy(lens).cuda()
    md = torch.from_numpy(m.astype(np.float32)).cuda()
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode=mode, kv_len=kl, attn_mask=md)
    dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode=mode, kv_len=kl,
                              attn_mask=md)
    torch.cuda.synchronize()
    ro, rl = oracle.attn_fwd(q, k, v, 1 / math.sqrt(D), causal, kv_len=lens, H=H, attn_mask=m)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H,
                                          attn_mask=m)
    o = o.reshape(B * H, S, D).cpu().numpy()
    assert_close(o, ro, mode, f"O mask {kind}")
    assert_close(l.cpu().numpy(), rl, mode, f"LSE mask {kind}")
    for got, ref, n in ((dq, rq, "dQ"), (dk, rk, "dK"), (dv, rv, "dV")):
        assert_close(got.reshape(B * H, S, D).cpu().numpy(), ref, mode, f"{n} mask {kind}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("nblk", [64, 200])
def test_attn_mask_blocked_key_prefix(mode, causal, D, nblk):
    """An additive mask that blocks (-1e30) whole leading key tiles, as left
    padding does: the kernels' softmax offset must not come from those
    tiles (a -1e30 level folded into the scores would absorb every later
    score). Under causal, rows that see only blocked keys are left unblocked
    (such a row has no unblocked key; the mirrors refuse it). Forward and
    backward against the oracle at the mode's bar."""
    from gonn_amd import hip
    B, H, Sq, Sk = 2, 2, 96 if not causal else 300, 300
    say(f"[masked] blocked prefix nblk={nblk} mode={mode} D={D} causal={causal}")
    rng = np.random.default_rng(1300 + nblk + D)
    m = rng.standard_normal((B, Sq, Sk)) * 0.5
    rows = np.arange(Sq) >= (nblk if causal else 0)
    m[:, rows, :nblk] = -1e30
    q, g = (randn((B * H, Sq, D), 1310 + i) for i in range(2))
    k, v = (randn((B * H, Sk, D), 1320 + i) for i in range(2))
    dev = [torch.from_numpy(x).cuda().reshape(B, H, -1, D) for x in (q, k, v, g)]
    md = torch.from_numpy(m.astype(np.float32)).cuda()
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode=mode, attn_mask=md)
    dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode=mode, attn_mask=md)
    torch.cuda.synchronize()
    ro, rl = oracle.attn_fwd(q, k, v, 1 / math.sqrt(D), causal, H=H, attn_mask=m)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, H=H, attn_mask=m)
    assert_close(o.reshape(B * H, Sq, D).cpu().numpy(), ro, mode, "O blocked prefix")
    assert_close(l.cpu().numpy(), rl, mode, "LSE blocked prefix")
    assert_close(dq.reshape(B * H, Sq, D).cpu().numpy(), rq, mode, "dQ blocked prefix")
    assert_close(dk.reshape(B * H, Sk, D).cpu().numpy(), rk, mode, "dK blocked prefix")
    assert_close(dv.reshape(B * H, Sk, D).cpu().numpy(), rv, mode, "dV blocked prefix")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_forward_masked_large_offset_mask(mode):
    """forward_masked with an additive mask carrying a large common offset
    per row (-1e4 + N(0,1)) and a blocked leading key band: the mirror shifts
    each row by its in-window maximum, so the fp32 scores keep their
    precision; against the oracle (fp64, GoNN's order of additions) at the
    mode's bar."""
    from gonn_amd import hip, nn
    E, H, B, T = 256, 4, 2, 150
    p = _params(E, 1400)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    x = randn((B, T, E), 1401).astype(np.float64)
    rng = np.random.default_rng(1402)
    m = rng.standard_normal((B, T, T)) - 1e4
    m[:, 70:, :66] = -1e30
    prev = hip.AttnMode()
    hip.SetAttnMode(mode)
    try:
        for causal in (False, True):
            say(f"[masked] large-offset mask mode={mode} causal={causal}")
            got = mha.forward_masked(x, x, x, causal=causal, attn_mask=m)
            ref = oracle.mha_fwd(x, x, x, p, H, causal=causal, attn_mask=m)
            assert_close(got, ref, mode, f"large-offset mask causal={causal}")
    finally:
        hip.SetAttnMode(prev)


@pytest.mark.parametrize("mode", ["fp32", "bf16", "f64"])
def test_forward_masked_blocked_rows_modes(mode):
    """forward_masked rows with no unblocked key, in each mode of the f64
    entries, cross-attention (Tq != Tk) included: GoNN's -1e30 terms absorb
    such a row's scores (a uniform average over the keys of the row's
    maximum summed mask, future keys included); the mirror passes them in
    the whole-row form, where the kernels' fp32 (or fp64) sums absorb the
    scores the same way. Against the oracle (fp64, GoNN's additions) at the
    mode's bar (f64: 1e-9, the reference's gate)."""
    from gonn_amd import hip, nn
    E, H, B, Tq, Tk = 256, 4, 3, 72, 136
    p = _params(E, 1500)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    x = randn((B, Tk, E), 1501).astype(np.float64)
    q = randn((B, Tq, E), 1502).astype(np.float64)
    pad = np.zeros((B, Tk))
    pad[0, :5] = 1      # padded leading keys
    pad[1] = 1          # every key padded
    pad[2, 100:] = 1    # a suffix
    am = randn((B, Tk, Tk), 1503).astype(np.float64)
    am[:, 7, :] = -1e30
    am[2, 0, 0] = -1e30
    prev = hip.AttnMode()
    hip.SetAttnMode(mode)
    try:
        for causal in (False, True):
            for (qq, kk, tag) in ((x, x, "self"), (q, x, "cross")):
                say(f"[masked] blocked rows mode={mode} causal={causal} {tag}")
                mk = am[:, :qq.shape[1], :kk.shape[1]]
                got = mha.forward_masked(qq, kk, kk, causal=causal, key_padding_mask=pad,
                                         attn_mask=np.ascontiguousarray(mk))
                ref = oracle.mha_fwd(qq, kk, kk, p, H, causal=causal, key_pad=pad, attn_mask=mk)
                if mode == "f64":
                    err = float(np.abs(got - ref).max())
                    say(f"[blocked rows f64] max_abs={err:.3e}")
                    assert err <= 1e-9, (tag, causal, err)
                else:
                    assert_close(got, ref, mode, f"blocked rows {tag} causal={causal}")
    finally:
        hip.SetAttnMode(prev)


def test_attn_mask_cross_attention_and_nn(mode="fp32"):
    """nn.MultiHeadAttention.forward_masked with an additive (B, Tq, Tk) mask
    on cross-attention, and fused_attn_diff with a (Tq, Tk) mask, against the
    oracle."""
    from gonn_amd import nn
    E, H, B, Tq, Tk = 256, 4, 2, 60, 130
    s = 1.0 / math.sqrt(E)
    p = {}
    for i, n in enumerate("qkvo"):
        p["W" + n] = randn((E, E), 890 + 2 * i).astype(np.float64) * s
        p["b" + n] = randn((E,), 891 + 2 * i).astype(np.float64) * 0.1
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    q = randn((B, Tq, E), 899).astype(np.float64)
    mem = randn((B, Tk, E), 900).astype(np.float64)
    m, _ = _mask_of("BTqTk", B, 1, Tq, Tk, 901)
    pad = np.zeros((B, Tk))
    pad[1, 90:] = 1
    got = mha.forward_masked(q, mem, mem, causal=True, key_padding_mask=pad, attn_mask=m)
    ref = oracle.mha_fwd(q, mem, mem, p, H, causal=True, key_pad=pad, attn_mask=m)
    assert_close(got, ref, "fp32", "forward_masked cross + attn_mask")

    S, D, BH = 80, 64, 4
    q2, k2, v2, g2 = (randn((BH, S, D), 910 + i) for i in range(4))
    m2, _ = _mask_of("TqTk", 1, 1, S, S, 915)
    O, node = nn.fused_attn_diff(q2, k2, v2, BH, S, D, 1 / math.sqrt(D), False, H=BH,
                                 attn_mask=m2)
    ro, _ = oracle.attn_fwd(q2, k2, v2, 1 / math.sqrt(D), False, H=BH, attn_mask=m2)
    assert_close(O.reshape(BH, S, D), ro, "fp32", "fused_attn_diff O attn_mask")
    grads = node(g2.ravel())
    ref = oracle.attn_bwd_autograd(q2, k2, v2, g2, causal=False, H=BH, attn_mask=m2)
    for got, r, n in zip(grads, ref, ("dQ", "dK", "dV")):
        assert_close(got.reshape(BH, S, D), r, "fp32", f"fused_attn_diff {n} attn_mask")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq_sk", [(70, 150), (150, 70)], ids=lambda t: f"{t[0]}x{t[1]}")
def test_cross_attention_backward_matches_oracle(mode, D, causal, sq_sk):
    """Cross-attention backward (Sq != Sk, top-left causal, key padding):
    dQ (B*H,Sq,D), dK, dV (B*H,Sk,D) against the oracle's autograd chain,
    in the stated mode (the bf16 backward packs K and V with their own key
    padding) at that mode's bar."""
    from gonn_amd import hip
    Sq, Sk = sq_sk
    B, H = 2, 2
    lens = np.array([Sk, Sk // 2 + 3], dtype=np.int32)
    say(f"[masked] cross bwd mode={mode} D={D} causal={causal} Sq={Sq} Sk={Sk}")
    q, g = (randn((B * H, Sq, D), 930 + i) for i in range(2))
    k, v = (randn((B * H, Sk, D), 932 + i) for i in range(2))
    dq_, dg_ = (torch.from_numpy(x).cuda().reshape(B, H, Sq, D) for x in (q, g))
    dk_, dv_ = (torch.from_numpy(x).cuda().reshape(B, H, Sk, D) for x in (k, v))
    kl = torch.from_numpy(lens).cuda()
    o, l = hip.attn_fwd(dq_, dk_, dv_, causal=causal, mode=mode, kv_len=kl)
    dq, dk, dv = hip.attn_bwd(dq_, dk_, dv_, o, l, dg_, causal=causal, mode=mode, kv_len=kl)
    torch.cuda.synchronize()
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H)
    assert dk.shape == dk_.shape and dq.shape == dq_.shape
    assert_close(dq.reshape(B * H, Sq, D).cpu().numpy(), rq, mode, "cross dQ")
    assert_close(dk.reshape(B * H, Sk, D).cpu().numpy(), rk, mode, "cross dK")
    assert_close(dv.reshape(B * H, Sk, D).cpu().numpy(), rv, mode, "cross dV")


def test_cross_attention_backward_f64_entry():
    """gonn_hip_flash_attn_f64_bwd_masked with Sq != Sk through
    FlashAttnF64BwdEx, with an additive (Sq, Sk) mask."""
    from gonn_amd import hip
    B, H, Sq, Sk, D = 2, 1, 40, 90, 64
    q, g = (randn((B * H, Sq, D), 940 + i) for i in range(2))
    k, v = (randn((B * H, Sk, D), 942 + i) for i in range(2))
    m, _ = _mask_of("TqTk", 1, 1, Sq, Sk, 944)
    sc = 1 / math.sqrt(D)
    O, L = hip.FlashAttnF64Ex(q, k, v, B, H, Sq, Sk, D, sc, True, lse=True, attn_mask=m)
    dq, dk, dv = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, B, H, Sq, D, sc, True, attn_mask=m, Sk=Sk)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=True, H=H, attn_mask=m)
    assert_close(dq.reshape(B * H, Sq, D), rq, "fp32", "f64 cross dQ")
    assert_close(dk.reshape(B * H, Sk, D), rk, "fp32", "f64 cross dK")
    assert_close(dv.reshape(B * H, Sk, D), rv, "fp32", "f64 cross dV")
