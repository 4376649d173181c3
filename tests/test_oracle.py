"""Pin the fp64 oracle (CPU only).

The reference's own attention path cannot run here (Go + CUDA, no toolchain),
and its golden file (nn/testdata/parity.golden:50-53) needs Go's math/rand
stream, which cannot be reproduced without Go. So every oracle function is
pinned by checks that do not retype its formula:
  * torch float64 (a library implementation) and the committed fixtures made
    from it (tests/golden/gen_golden.py);
  * a long-double brute force;
  * closed forms (Sk=1 -> O=V, Q=0 -> prefix mean, LSE of equal scores);
  * the reference's masked-attention invariants (nn/attention_masked_test.go);
  * the reference's refAttn (benchmark/flashattn/main.go:39-75) restated;
  * central finite differences with the reference's flashbwd protocol
    (benchmark/flashbwd/main.go:40-95) and its nn gradcheck tolerance
    (nn/gradcheck_test.go:72-75);
and each planted mistake (oracle.set_mutation) must make one of them fail.
"""
import math
import os

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_golden.npz")


@pytest.fixture(autouse=True)
def _no_mutation():
    oracle.set_mutation("none")
    yield
    oracle.set_mutation("none")


def _golden_cases():
    z = np.load(GOLD, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def _torch_fwd(q, k, v, scale, causal, kv_len=None, H=1):
    tq, tk, tv = (torch.from_numpy(np.asarray(x, np.float64)) for x in (q, k, v))
    s = (tq @ tk.transpose(1, 2)) * scale
    Sq, Sk = s.shape[1], s.shape[2]
    if causal:
        s = s + torch.where(torch.arange(Sk)[None, :] > torch.arange(Sq)[:, None], -1e30, 0.0)
    if kv_len is not None:
        for bh in range(s.shape[0]):
            s[bh, :, kv_len[bh // H]:] += -1e30
    return (torch.softmax(s, -1) @ tv).numpy(), torch.logsumexp(s, -1).numpy()


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------
def test_fwd_matches_golden_fixtures():
    z, names = _golden_cases()
    assert len(names) >= 8
    for n in names:
        BH, Sq, Sk, D, causal, H = (int(x) for x in z[n + "/meta"])
        kv = z[n + "/kv_len"] if (n + "/kv_len") in z.files else None
        O, L = oracle.attn_fwd(z[n + "/q"], z[n + "/k"], z[n + "/v"], causal=bool(causal),
                               kv_len=kv, H=H)
        np.testing.assert_allclose(O, z[n + "/O"], atol=1e-12, rtol=0, err_msg=n)
        np.testing.assert_allclose(L, z[n + "/LSE"], atol=1e-12, rtol=0, err_msg=n)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(3, 37, 37, 64), (2, 65, 130, 128), (2, 130, 65, 32)])
def test_fwd_matches_torch_fp64(causal, shape):
    BH, Sq, Sk, D = shape
    rng = np.random.default_rng(sum(shape) + causal)
    q, k, v = rng.standard_normal((BH, Sq, D)), rng.standard_normal((BH, Sk, D)), \
        rng.standard_normal((BH, Sk, D))
    O, L = oracle.attn_fwd(q, k, v, causal=causal)
    to, tl = _torch_fwd(q, k, v, 1 / math.sqrt(D), causal)
    np.testing.assert_allclose(O, to, atol=1e-12, rtol=0)
    np.testing.assert_allclose(L, tl, atol=1e-12, rtol=0)
    # torch's fused SDPA (a second library path) for the square case
    if Sq == Sk:
        ref = torch.nn.functional.scaled_dot_product_attention(
            *(torch.from_numpy(x) for x in (q, k, v)), is_causal=causal).numpy()
        np.testing.assert_allclose(O, ref, atol=1e-12, rtol=0)


def test_fwd_long_double_brute_force():
    rng = np.random.default_rng(3)
    BH, S, D = 2, 9, 8
    q, k, v = (rng.standard_normal((BH, S, D)) for _ in range(3))
    O, L = oracle.attn_fwd(q, k, v, causal=True)
    ql, kl, vl = (x.astype(np.longdouble) for x in (q, k, v))
    sc = np.longdouble(1) / np.sqrt(np.longdouble(D))
    for bh in range(BH):
        for i in range(S):
            s = np.array([np.dot(ql[bh, i], kl[bh, j]) * sc for j in range(i + 1)])
            w = np.exp(s - s.max())
            ref = (w[:, None] * vl[bh, :i + 1]).sum(0) / w.sum()
            assert np.max(np.abs(O[bh, i] - ref.astype(np.float64))) < 1e-14
            assert abs(L[bh, i] - float(s.max() + np.log(w.sum()))) < 1e-14


def test_fwd_refattn_restatement():
    """oracle.ref_attn restates refAttn (benchmark/flashattn/main.go:39-75);
    the fused kernel was held to 1e-9 against it; the oracle matches it to
    rounding."""
    rng = np.random.default_rng(7)
    BH, S, d = 3, 12, 8
    q, k, v = (rng.standard_normal((BH, S, d)) for _ in range(3))
    for causal in (False, True):
        O, _ = oracle.attn_fwd(q, k, v, causal=causal)
        np.testing.assert_allclose(O, oracle.ref_attn(q, k, v, 1 / math.sqrt(d), causal),
                                   atol=1e-14, rtol=0)


def test_fwd_closed_forms():
    rng = np.random.default_rng(11)
    BH, S, D = 2, 50, 16
    q, k, v = (rng.standard_normal((BH, S, D)) for _ in range(3))
    # Sk = 1: the single key gets weight 1, O = V, LSE = scaled score
    O, L = oracle.attn_fwd(q, k[:, :1], v[:, :1], causal=False)
    assert np.array_equal(O, np.broadcast_to(v[:, :1], O.shape))
    np.testing.assert_allclose(L, (q @ k[:, :1].transpose(0, 2, 1))[..., 0] / 4.0, atol=1e-14)
    # Q = 0: uniform weights over the causal prefix; LSE = ln(i+1)
    O, L = oracle.attn_fwd(np.zeros_like(q), k, v, causal=True)
    ref = np.cumsum(v, axis=1) / np.arange(1, S + 1)[None, :, None]
    np.testing.assert_allclose(O, ref, atol=1e-14)
    np.testing.assert_allclose(L, np.broadcast_to(np.log(np.arange(1, S + 1)), L.shape),
                               atol=1e-14)
    # outputs are convex combinations of V rows
    O, _ = oracle.attn_fwd(q, k, v, causal=True)
    for bh in range(BH):
        for i in range(S):
            assert np.all(O[bh, i] <= v[bh, :i + 1].max(0) + 1e-12)
            assert np.all(O[bh, i] >= v[bh, :i + 1].min(0) - 1e-12)


def test_fwd_masked_invariants():
    """nn/attention_masked_test.go:42-81 adapted: keys the mask removes (future
    keys under the causal mask, padded keys) do not change the output at all."""
    rng = np.random.default_rng(13)
    BH, S, D = 4, 10, 8
    q, k, v = (rng.standard_normal((BH, S, D)) for _ in range(3))
    O, L = oracle.attn_fwd(q, k, v, causal=True)
    k2, v2 = k.copy(), v.copy()
    p = 6
    k2[:, p + 1:] += 7.5
    v2[:, p + 1:] -= 3.25
    O2, L2 = oracle.attn_fwd(q, k2, v2, causal=True)
    assert np.array_equal(O[:, :p + 1], O2[:, :p + 1])
    assert np.array_equal(L[:, :p + 1], L2[:, :p + 1])
    assert not np.array_equal(O[:, p + 1:], O2[:, p + 1:])
    # key padding: per-batch lengths (H=2 heads per batch)
    lens = np.array([3, 8], np.int32)
    O, _ = oracle.attn_fwd(q, k, v, causal=False, kv_len=lens, H=2)
    k3, v3 = k.copy(), v.copy()
    for b in range(2):
        k3[2 * b:2 * b + 2, lens[b]:] *= -2
        v3[2 * b:2 * b + 2, lens[b]:] += 11
    O3, _ = oracle.attn_fwd(q, k3, v3, causal=False, kv_len=lens, H=2)
    assert np.array_equal(O, O3)
    # ...and padding a key equals dropping it
    for b in range(2):
        sl = slice(2 * b, 2 * b + 2)
        Ot, _ = oracle.attn_fwd(q[sl], k[sl, :lens[b]], v[sl, :lens[b]], causal=False)
        np.testing.assert_allclose(O[sl], Ot, atol=1e-15)


def test_fwd_rows_subset_is_identical():
    rng = np.random.default_rng(17)
    q, k, v = (rng.standard_normal((2, 40, 16)) for _ in range(3))
    O, L = oracle.attn_fwd(q, k, v, causal=True)
    rows = np.array([0, 5, 39])
    Or, Lr = oracle.attn_fwd(q, k, v, causal=True, rows=rows)
    assert np.array_equal(O[:, rows], Or[:, rows]) and np.array_equal(L[:, rows], Lr[:, rows])


@pytest.mark.parametrize("causal", [False, True])
def test_goflow_baseline_equals_oracle(causal):
    """The timed CPU baseline (GoNN's pass structure: whole-tensor passes,
    materialised broadcasts) computes the same fp64 numbers as the oracle:
    the same op order per element, so bit for bit."""
    rng = np.random.default_rng(18)
    q, k, v = (rng.standard_normal((3, 70, 32)) for _ in range(3))
    O = oracle.attn_fwd_goflow(q, k, v, scale=0.3, causal=causal)
    Or, _ = oracle.attn_fwd(q, k, v, scale=0.3, causal=causal)
    assert np.array_equal(O, Or)


# ---------------------------------------------------------------------------
# backward
# ---------------------------------------------------------------------------
def test_bwd_matches_golden_fixtures():
    z, names = _golden_cases()
    for n in names:
        BH, Sq, Sk, D, causal, H = (int(x) for x in z[n + "/meta"])
        if Sq != Sk or (n + "/kv_len") in z.files:
            continue
        dQ, dK, dV = oracle.attn_bwd_autograd(z[n + "/q"], z[n + "/k"], z[n + "/v"],
                                              z[n + "/dO"], causal=bool(causal))
        for nm, got in (("dQ", dQ), ("dK", dK), ("dV", dV)):
            np.testing.assert_allclose(got, z[n + "/" + nm], atol=1e-12, rtol=0,
                                       err_msg=f"{n} {nm}")


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_matches_torch_autograd(causal):
    rng = np.random.default_rng(19 + causal)
    BH, S, D = 3, 45, 64
    q, k, v, g = (rng.standard_normal((BH, S, D)) for _ in range(4))
    dQ, dK, dV = oracle.attn_bwd_autograd(q, k, v, g, causal=causal)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).backward(
        torch.tensor(g))
    for got, t in ((dQ, tq), (dK, tk), (dV, tv)):
        np.testing.assert_allclose(got, t.grad.numpy(), atol=1e-12, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_key_padding_matches_torch_autograd(causal):
    """ForwardMasked's key padding in the backward: torch fp64 autograd through
    the same additive -1e30 masks (a library path), exact zeros on padded keys,
    and kv_len = S equal to no padding bit for bit."""
    rng = np.random.default_rng(23 + causal)
    B, H, S, D = 3, 2, 40, 64
    lens = [40, 17, 1]
    q, k, v, g = (rng.standard_normal((B * H, S, D)) for _ in range(4))
    dQ, dK, dV = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    s = (tq @ tk.transpose(1, 2)) / math.sqrt(D)
    mask = torch.zeros(B * H, S, S, dtype=torch.float64)
    if causal:
        mask += torch.where(torch.arange(S)[None, :] > torch.arange(S)[:, None], -1e30, 0.0)
    for bh in range(B * H):
        mask[bh, :, lens[bh // H]:] += -1e30
    (torch.softmax(s + mask, -1) @ tv).backward(torch.tensor(g))
    for got, t in ((dQ, tq), (dK, tk), (dV, tv)):
        np.testing.assert_allclose(got, t.grad.numpy(), atol=1e-12, rtol=0)
    for bh in range(B * H):
        n = lens[bh // H]
        assert np.all(dK[bh, n:] == 0.0) and np.all(dV[bh, n:] == 0.0)
    full = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=[S] * B, H=H)
    plain = oracle.attn_bwd_autograd(q, k, v, g, causal=causal)
    for a, b in zip(full, plain):
        assert np.array_equal(a, b)


def _fd_check(causal, fwd=oracle.attn_fwd, bwd=None):
    """benchmark/flashbwd/main.go:40-95: BH=2, S=6, D=64, loss = sum(O*dO),
    eps=1e-6, indices {0,1,64,130,200,n-1}, relErr <= 1e-4."""
    rng = np.random.default_rng(1)
    BH, S, D = 2, 6, 64
    n = BH * S * D
    Q, K, V, dO = (rng.standard_normal(n) for _ in range(4))
    shp = (BH, S, D)
    dQ, dK, dV = (bwd or (lambda *a: oracle.attn_bwd_autograd(*a, causal=causal)))(
        Q.reshape(shp), K.reshape(shp), V.reshape(shp), dO.reshape(shp))
    eps = 1e-6
    worst = 0.0

    def loss():
        O, _ = fwd(Q.reshape(shp), K.reshape(shp), V.reshape(shp), causal=causal)
        return float(np.sum(O.ravel() * dO))

    for x, ana in ((Q, dQ), (K, dK), (V, dV)):
        for idx in (0, 1, 64, 130, 200, n - 1):
            save = x[idx]
            x[idx] = save + eps
            lp = loss()
            x[idx] = save - eps
            lm = loss()
            x[idx] = save
            num = (lp - lm) / (2 * eps)
            ag = ana.ravel()[idx]
            worst = max(worst, abs(num - ag) / (abs(num) + abs(ag) + 1e-9))
    return worst


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_finite_differences_flashbwd_protocol(causal):
    assert _fd_check(causal) <= 1e-4


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_rows_equals_autograd_chain(causal):
    rng = np.random.default_rng(23)
    BH, S, D = 2, 33, 32
    q, k, v, g = (rng.standard_normal((BH, S, D)) for _ in range(4))
    O, L = oracle.attn_fwd(q, k, v, causal=causal)
    full = oracle.attn_bwd_autograd(q, k, v, g, causal=causal)
    rows = np.arange(S)
    part = oracle.attn_bwd_rows(q, k, v, O, L, g, causal=causal, qrows=rows, krows=rows)
    for a, b in zip(part, full):
        np.testing.assert_allclose(a, b, atol=1e-12, rtol=0)


# ---------------------------------------------------------------------------
# MultiHeadAttention composition (projections + core)
# ---------------------------------------------------------------------------
def _mha_params(E, rng):
    s = 1 / math.sqrt(E)
    return {n: rng.standard_normal((E, E)) * s if n.startswith("W") else rng.standard_normal(E) * s
            for n in ("Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo")}


@pytest.mark.parametrize("causal", [False, True])
def test_mha_matches_torch_multi_head_attention(causal):
    """C1 shape (B=2, S=128, E=256, H=4) against torch's fp64 MHA forward."""
    rng = np.random.default_rng(29)
    B, T, E, H = 2, 128, 256, 4
    x = rng.standard_normal((B, T, E)) / math.sqrt(E)
    p = _mha_params(E, rng)
    ours = oracle.mha_fwd(x, x, x, p, H, causal=causal)
    tx = torch.from_numpy(x).transpose(0, 1)
    mask = torch.triu(torch.full((T, T), -1e30, dtype=torch.float64), 1) if causal else None
    ref, _ = torch.nn.functional.multi_head_attention_forward(
        tx, tx, tx, E, H, None, torch.from_numpy(np.concatenate([p["bq"], p["bk"], p["bv"]])),
        None, None, False, 0.0, torch.from_numpy(p["Wo"]), torch.from_numpy(p["bo"]),
        training=False, need_weights=False, attn_mask=mask, use_separate_proj_weight=True,
        q_proj_weight=torch.from_numpy(p["Wq"]), k_proj_weight=torch.from_numpy(p["Wk"]),
        v_proj_weight=torch.from_numpy(p["Wv"]))
    np.testing.assert_allclose(ours, ref.transpose(0, 1).numpy(), atol=1e-12, rtol=0)


def test_mha_key_padding_matches_torch():
    rng = np.random.default_rng(31)
    B, T, E, H = 2, 12, 32, 4
    x = rng.standard_normal((B, T, E))
    p = _mha_params(E, rng)
    pad = np.zeros((B, T))
    pad[0, 9:] = 1
    pad[1, 4:] = 1
    ours = oracle.mha_fwd(x, x, x, p, H, key_pad=pad)
    tx = torch.from_numpy(x).transpose(0, 1)
    ref, _ = torch.nn.functional.multi_head_attention_forward(
        tx, tx, tx, E, H, None, torch.from_numpy(np.concatenate([p["bq"], p["bk"], p["bv"]])),
        None, None, False, 0.0, torch.from_numpy(p["Wo"]), torch.from_numpy(p["bo"]),
        training=False, need_weights=False, key_padding_mask=torch.from_numpy(pad != 0),
        use_separate_proj_weight=True, q_proj_weight=torch.from_numpy(p["Wq"]),
        k_proj_weight=torch.from_numpy(p["Wk"]), v_proj_weight=torch.from_numpy(p["Wv"]))
    np.testing.assert_allclose(ours, ref.transpose(0, 1).numpy(), atol=1e-12, rtol=0)


# ---------------------------------------------------------------------------
# planted mistakes: each must be caught by one of the checks above
# ---------------------------------------------------------------------------
def _fwd_vs_torch(causal=True, D=16, S=16, big=1.0):
    rng = np.random.default_rng(37)
    q, k, v = (rng.standard_normal((2, S, D)) * big for _ in range(3))
    O, L = oracle.attn_fwd(q, k, v, causal=causal)
    to, tl = _torch_fwd(q, k, v, 1 / math.sqrt(D), causal)
    ok_o = np.all(np.isfinite(O)) and np.max(np.abs(O - to)) < 1e-9
    ok_l = np.all(np.isfinite(L)) and np.max(np.abs(L - tl)) < 1e-9
    return ok_o and ok_l


@pytest.mark.parametrize("mutation", ["no_scale", "causal_ge", "transpose_v", "lse_log2",
                                      "no_max_sub", "ds_sign"])
def test_planted_mistakes_are_caught(mutation):
    assert _fwd_vs_torch() and _fwd_vs_torch(big=40.0) and _fd_check(True) <= 1e-4
    oracle.set_mutation(mutation)
    caught = (not _fwd_vs_torch()) or (not _fwd_vs_torch(big=40.0))
    if mutation == "ds_sign":
        rng = np.random.default_rng(41)
        q, k, v, g = (rng.standard_normal((2, 9, 8)) for _ in range(4))
        O, L = oracle.attn_fwd(q, k, v, causal=True)
        part = oracle.attn_bwd_rows(q, k, v, O, L, g, causal=True, qrows=np.arange(9),
                                    krows=np.arange(9))
        full = oracle.attn_bwd_autograd(q, k, v, g, causal=True)
        caught = caught or not all(np.allclose(a, b, atol=1e-9) for a, b in zip(part, full))
    assert caught, f"planted mistake {mutation} went unnoticed"


@pytest.mark.parametrize("shape_kind", ["TqTk", "BTqTk", "BHTqTk3", "BHTqTk4"])
def test_additive_attn_mask_matches_torch(shape_kind):
    """WithAttnMask (nn/attention.go:212-257) in the forward and the autograd
    chain: torch fp64 through scores*scale + causal + mask + key padding, for
    each of expandAttnMask's accepted shapes."""
    rng = np.random.default_rng(31)
    B, H, S, D = 2, 3, 24, 64
    q, k, v, g = (rng.standard_normal((B * H, S, D)) for _ in range(4))
    full = rng.standard_normal((B, H, S, S)) * 2.0
    full[..., 5] = -1e30  # a blocked key column, as the reference suggests
    m = {"TqTk": full[0, 0], "BTqTk": full[:, 0], "BHTqTk3": full.reshape(B * H, S, S),
         "BHTqTk4": full}[shape_kind]
    dense = np.broadcast_to(m.reshape((1, 1, S, S)) if m.ndim == 2 else
                            (m.reshape(B, 1, S, S) if shape_kind == "BTqTk" else m.reshape(B, H, S, S)),
                            (B, H, S, S)).reshape(B * H, S, S)
    lens = [S, 17]
    O, L = oracle.attn_fwd(q, k, v, causal=True, kv_len=lens, H=H, attn_mask=m)
    dq, dk, dv = oracle.attn_bwd_autograd(q, k, v, g, causal=True, kv_len=lens, H=H, attn_mask=m)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    s = (tq @ tk.transpose(1, 2)) / math.sqrt(D)
    s = s + torch.where(torch.arange(S)[None, :] > torch.arange(S)[:, None], -1e30, 0.0)
    s = s + torch.from_numpy(np.array(dense))
    pad = torch.zeros(B * H, 1, S, dtype=torch.float64)
    for bh in range(B * H):
        pad[bh, :, lens[bh // H]:] = -1e30
    s = s + pad
    out = torch.softmax(s, -1) @ tv
    np.testing.assert_allclose(O, out.detach().numpy(), atol=1e-12, rtol=0)
    np.testing.assert_allclose(L, torch.logsumexp(s, -1).detach().numpy(), atol=1e-9, rtol=0)
    out.backward(torch.tensor(g))
    for got, t in ((dq, tq), (dk, tk), (dv, tv)):
        np.testing.assert_allclose(got, t.grad.numpy(), atol=1e-12, rtol=0)
    with pytest.raises(ValueError):
        oracle.attn_fwd(q, k, v, attn_mask=np.zeros((S, S + 1)), H=H)


@pytest.mark.parametrize("causal", [False, True])
def test_cross_attention_backward_matches_torch(causal):
    """Cross-attention (Sq != Sk, top-left causal as causalMaskAdd builds it,
    nn/attention.go:185-196) through the autograd chain, with key padding:
    torch fp64 autograd through the same masks."""
    rng = np.random.default_rng(37 + causal)
    B, H, Sq, Sk, D = 2, 2, 21, 53, 64
    q, g = (rng.standard_normal((B * H, Sq, D)) for _ in range(2))
    k, v = (rng.standard_normal((B * H, Sk, D)) for _ in range(2))
    lens = [53, 30]
    dq, dk, dv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    s = (tq @ tk.transpose(1, 2)) / math.sqrt(D)
    if causal:
        s = s + torch.where(torch.arange(Sk)[None, :] > torch.arange(Sq)[:, None], -1e30, 0.0)
    pad = torch.zeros(B * H, 1, Sk, dtype=torch.float64)
    for bh in range(B * H):
        pad[bh, :, lens[bh // H]:] = -1e30
    (torch.softmax(s + pad, -1) @ tv).backward(torch.tensor(g))
    for got, t in ((dq, tq), (dk, tk), (dv, tv)):
        np.testing.assert_allclose(got, t.grad.numpy(), atol=1e-12, rtol=0)
