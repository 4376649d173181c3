"""GPU parity of the flash backward (dQ, dK, dV) against the fp64 oracle,
through the C ABI.

The oracle's gradients are GoNN's autograd chain through the pure-Go core
(attn_bwd_autograd) or, at full size, its closed form on sampled rows
(attn_bwd_rows, the identities of backend/cuda/gonn_cuda.cu:333-340); both are
pinned in test_oracle.py. O and LSE fed to the GPU backward come from the GPU
forward of the same mode, as in a training step.

Cases: small ragged shapes for both modes, D in {64, 128}, causal and not;
signed and zero scales; many queries against a handful of keys; the golden
fixtures and the reference's flashbwd shape through the f64 entry point;
BASELINE config C5 (B=2 H=16 S=8192 D=128 causal, bf16) on sampled rows plus
size-independent identities on the full output.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _fwd_bwd(q, k, v, g, causal, mode, scale=None):
    from gonn_amd import hip
    dq_, dk_, dv_, dg_ = _dev(q), _dev(k), _dev(v), _dev(g)
    o, l = hip.attn_fwd(dq_, dk_, dv_, causal=causal, mode=mode, scale=scale)
    dq, dk, dv = hip.attn_bwd(dq_, dk_, dv_, o, l, dg_, causal=causal, mode=mode, scale=scale)
    torch.cuda.synchronize()
    return (o.cpu().numpy(), l.cpu().numpy(), dq.cpu().numpy(), dk.cpu().numpy(),
            dv.cpu().numpy())


SMALL = [(1, 1), (2, 7), (3, 37), (2, 64), (2, 128), (2, 129), (1, 200), (2, 300)]


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "x".join(map(str, s)))
def test_bwd_small(mode, D, causal, shape):
    BH, S = shape
    seed = 3000 + 11 * BH + S + D + int(causal)
    q, k, v, g = (randn((BH, S, D), seed + i) for i in range(4))
    say(f"bwd_small mode={mode} D={D} causal={causal} shape={shape}")
    _, _, dq, dk, dv = _fwd_bwd(q, k, v, g, causal, mode)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal)
    assert_close(dq, rq, mode, "dQ")
    assert_close(dk, rk, mode, "dK")
    assert_close(dv, rv, mode, "dV")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_bwd_scale_variants(mode):
    """Negative and zero scales: gradients of softmax(scale QK^T) V.

    The bf16 bar (2e-2 + 1e-2|ref|) is stated for scale = 1/sqrt(D); the
    error of bf16-rounded scores grows with |scale| * sqrt(D) (at -0.2 with
    D = 64 it reaches 2.1e-2 on dK), so bf16 is checked at |scale| <= 1/sqrt(D).
    """
    BH, S, D = 2, 150, 64
    q, k, v, g = (randn((BH, S, D), 50 + i) for i in range(4))
    for scale in ((-0.2, 0.0, 0.05) if mode == "fp32" else (-0.125, 0.0, 0.05)):
        say(f"bwd scale={scale} mode={mode}")
        _, _, dq, dk, dv = _fwd_bwd(q, k, v, g, True, mode, scale=scale)
        rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, scale=scale, causal=True)
        assert_close(dq, rq, mode, f"dQ scale={scale}")
        assert_close(dk, rk, mode, f"dK scale={scale}")
        assert_close(dv, rv, mode, f"dV scale={scale}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", ["self", "kv_len", "mask"])
def test_bwd_bf16_dq_paths(D, causal, case, monkeypatch):
    """The bf16 backward's two dQ paths: dQ from the dS the dK/dV kernel
    stores (the default) and dQ with S and dP formed a second time
    (GONN_HIP_BWD_DQ=recompute). Both are held to the bf16 bar against the
    oracle, with key
    padding and an additive mask; dK and dV come from the same kernel on
    either path and agree bitwise."""
    from gonn_amd import hip
    from tests.test_gpu_masked import _mask_of
    B, H, S = 2, 2, 300
    lens = np.array([300, 171], dtype=np.int32) if case != "self" else None
    m = _mask_of("BHTqTk4", B, H, S, S, 77)[0] if case == "mask" else None
    q, k, v, g = (randn((B * H, S, D), 4100 + D + i) for i in range(4))
    dev = [torch.from_numpy(x).cuda().reshape(B, H, S, D) for x in (q, k, v, g)]
    kl = torch.from_numpy(lens).cuda() if lens is not None else None
    md = torch.from_numpy(m.astype(np.float32)).cuda() if m is not None else None
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode="bf16", kv_len=kl, attn_mask=md)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H,
                                          attn_mask=m)
    got = {}
    for path in ("ds", "recompute"):
        if path == "recompute":
            monkeypatch.setenv("GONN_HIP_BWD_DQ", "recompute")
        else:
            monkeypatch.delenv("GONN_HIP_BWD_DQ", raising=False)
        say(f"bwd dq path={path} D={D} causal={causal} case={case}")
        dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode="bf16",
                                  kv_len=kl, attn_mask=md)
        torch.cuda.synchronize()
        got[path] = [x.reshape(B * H, S, D).cpu().numpy() for x in (dq, dk, dv)]
        for x, ref, n in zip(got[path], (rq, rk, rv), ("dQ", "dK", "dV")):
            assert_close(x, ref, "bf16", f"{n} path={path}")
    assert np.array_equal(got["ds"][1], got["recompute"][1])
    assert np.array_equal(got["ds"][2], got["recompute"][2])


@pytest.mark.parametrize("shape", [(100, 300), (300, 100), (129, 520)],
                         ids=lambda s: f"Sq{s[0]}xSk{s[1]}")
@pytest.mark.parametrize("causal", [False, True])
def test_bwd_bf16_dq_paths_cross(shape, causal, monkeypatch):
    """Sq != Sk on both bf16 dQ paths (top-left causal): with Sk > Sq the
    causal key blocks past every query store no dS blocks and the dQ kernel
    never reads them; with Sq > Sk every key block reaches the later
    queries. Both paths against the oracle, dK/dV bitwise equal."""
    from gonn_amd import hip
    Sq, Sk = shape
    B, H, D = 1, 2, 128
    q = randn((B * H, Sq, D), 4300 + Sq)
    k, v = (randn((B * H, Sk, D), 4301 + Sk + i) for i in range(2))
    g = randn((B * H, Sq, D), 4305 + Sq)
    dev = [torch.from_numpy(x).cuda().reshape(B, H, x.shape[1], D) for x in (q, k, v, g)]
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode="bf16")
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal)
    got = {}
    for path in ("ds", "recompute"):
        if path == "recompute":
            monkeypatch.setenv("GONN_HIP_BWD_DQ", "recompute")
        else:
            monkeypatch.delenv("GONN_HIP_BWD_DQ", raising=False)
        say(f"bwd dq path={path} Sq={Sq} Sk={Sk} causal={causal}")
        dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode="bf16")
        torch.cuda.synchronize()
        got[path] = [x.reshape(B * H, -1, D).cpu().numpy() for x in (dq, dk, dv)]
        for x, ref, n in zip(got[path], (rq, rk, rv), ("dQ", "dK", "dV")):
            assert_close(x, ref, "bf16", f"{n} path={path}")
    assert np.array_equal(got["ds"][1], got["recompute"][1])
    assert np.array_equal(got["ds"][2], got["recompute"][2])


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", ["self", "kv_len", "mask", "Sq>Sk", "Sq<Sk"])
def test_bwd_bf16_ds_chunks_bit_exact(D, causal, case, monkeypatch):
    """The dS path in key-block chunks (GONN_HIP_BWD_DS_MB below the call's
    dS): each chunk's dK/dV stores its dS and the dQ kernel adds the chunk's
    keys to dQ, from the fp32 partial the previous chunk stored, with the
    scale on the last chunk only. The MFMAs accumulate the same products in
    the same order, so dQ, dK and dV equal the one-chunk call's bit for bit.
    Budgets of 3 MB (two 128-key blocks a chunk at 1000 keys) and 0.25 MB
    (one block a chunk, and causal chunks past every query holding no
    blocks); the chunked result also against the oracle."""
    from gonn_amd import hip
    from tests.test_gpu_masked import _mask_of
    B, H = 2, 3
    Sq, Sk = {"Sq>Sk": (900, 400), "Sq<Sk": (400, 900)}.get(case, (1000, 1000))
    lens = np.array([Sk, 3 * Sk // 5], dtype=np.int32) if case == "kv_len" else None
    m = _mask_of("BHTqTk4", B, H, Sq, Sk, 78)[0] if case == "mask" else None
    q, g = (randn((B * H, Sq, D), 4500 + D + i) for i in range(2))
    k, v = (randn((B * H, Sk, D), 4510 + D + i) for i in range(2))
    dev = [torch.from_numpy(x).cuda().reshape(B, H, x.shape[1], D) for x in (q, k, v, g)]
    kl = torch.from_numpy(lens).cuda() if lens is not None else None
    md = torch.from_numpy(m.astype(np.float32)).cuda() if m is not None else None
    monkeypatch.delenv("GONN_HIP_BWD_DQ", raising=False)
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode="bf16", kv_len=kl, attn_mask=md)
    got = {}
    for mb in (None, "3", "0.25"):
        if mb is None:
            monkeypatch.delenv("GONN_HIP_BWD_DS_MB", raising=False)
        else:
            monkeypatch.setenv("GONN_HIP_BWD_DS_MB", mb)
        say(f"bwd dS chunks budget={mb} MB D={D} causal={causal} case={case}")
        dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode="bf16",
                                  kv_len=kl, attn_mask=md)
        torch.cuda.synchronize()
        got[mb] = [x.reshape(B * H, -1, D).cpu().numpy() for x in (dq, dk, dv)]
    monkeypatch.delenv("GONN_HIP_BWD_DS_MB", raising=False)
    for mb in ("3", "0.25"):
        for a, b, n in zip(got[mb], got[None], ("dQ", "dK", "dV")):
            assert np.array_equal(a, b), (n, mb, float(np.abs(a - b).max()))
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal, kv_len=lens, H=H,
                                          attn_mask=m)
    live = np.ones(B * H, bool) if lens is None else np.repeat(lens > 0, H)
    for x, ref, n in zip(got["0.25"], (rq, rk, rv), ("dQ", "dK", "dV")):
        assert_close(x[live], ref[live], "bf16", f"{n} in chunks")


@pytest.mark.parametrize("i", range(24))
def test_bwd_bf16_ds_chunks_random(i, monkeypatch):
    """The random sweep's shapes and options (tests/test_gpu_random.py: ragged
    Sq and Sk, cross-attention, causal, key padding with empty sequences,
    every mask shape), bf16 mode: the dS path cut into one-key-block chunks
    by a 0.03 MB budget gives dQ, dK and dV bit-identical to one pass."""
    from gonn_amd import hip
    import tests.test_gpu_random as R
    c = R._case(i)
    B, H, D, Sq, Sk = c["B"], c["H"], c["D"], c["Sq"], c["Sk"]
    r = np.random.default_rng(c["seed"])
    q, g = (r.standard_normal((B * H, Sq, D)) for _ in range(2))
    k, v = (r.standard_normal((B * H, Sk, D)) for _ in range(2))
    m = R._mask(c["mkind"], B, H, Sq, Sk, r) if c["mkind"] else None
    dev = lambda x, S: torch.from_numpy(x.astype(np.float32)).cuda().reshape(B, H, S, D)  # noqa: E731
    dq_, dk_, dv_, dg_ = dev(q, Sq), dev(k, Sk), dev(v, Sk), dev(g, Sq)
    kl = torch.from_numpy(c["kv"]).cuda() if c["kv"] is not None else None
    md = torch.from_numpy(m.astype(np.float32)).cuda() if m is not None else None
    say(f"[chunks random {i}] B={B} H={H} D={D} Sq={Sq} Sk={Sk} causal={c['causal']} "
        f"kv={None if c['kv'] is None else list(c['kv'])} mask={c['mkind']}")
    o, l = hip.attn_fwd(dq_, dk_, dv_, causal=c["causal"], mode="bf16", kv_len=kl, attn_mask=md)
    got = []
    for budget in (None, "0.03"):
        monkeypatch.delenv("GONN_HIP_BWD_DQ", raising=False)
        if budget is None:
            monkeypatch.delenv("GONN_HIP_BWD_DS_MB", raising=False)
        else:
            monkeypatch.setenv("GONN_HIP_BWD_DS_MB", budget)
        gr = hip.attn_bwd(dq_, dk_, dv_, o, l, dg_, causal=c["causal"], mode="bf16", kv_len=kl,
                          attn_mask=md)
        torch.cuda.synchronize()
        got.append([t.cpu() for t in gr])
    for n, a, b in zip(("dQ", "dK", "dV"), *got):
        assert torch.equal(a, b), n


@pytest.mark.parametrize("path", ["ds", "recompute"])
def test_bwd_bf16_full_rows_many_key_blocks(path, monkeypatch):
    """B=1 H=2 S=4096 D=128 causal, bf16 MFMA: every row of dQ, dK and dV
    against the oracle's autograd chain. 32 key blocks of 128 keys reach
    2 to 64 query tiles each, so the compact causal dS placement
    (ds_block_base) is checked on every block, not on sampled rows, on
    both dQ paths."""
    from gonn_amd import hip
    B, H, S, D = 1, 2, 4096, 128
    q, k, v, g = (randn((B * H, S, D), 4400 + i) for i in range(4))
    dev = [torch.from_numpy(x).cuda() for x in (q, k, v, g)]
    if path == "recompute":
        monkeypatch.setenv("GONN_HIP_BWD_DQ", "recompute")
    else:
        monkeypatch.delenv("GONN_HIP_BWD_DQ", raising=False)
    say(f"bwd full rows S={S} path={path}")
    o, l = hip.attn_fwd(*dev[:3], causal=True, mode="bf16")
    dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=True, mode="bf16")
    torch.cuda.synchronize()
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=True)
    assert_close(dq.cpu().numpy(), rq, "bf16", f"dQ path={path}")
    assert_close(dk.cpu().numpy(), rk, "bf16", f"dK path={path}")
    assert_close(dv.cpu().numpy(), rv, "bf16", f"dV path={path}")


@pytest.mark.parametrize("D,causal", [(128, True), (64, False), (64, True)])
def test_bwd_fp32_full_rows_many_blocks(D, causal):
    """fp32-MFMA mode, B=1 H=2 S=1536: every row of dQ, dK and dV against
    the oracle's autograd chain at the fp32 bar (1e-4). 1536 rows span 12
    key blocks and 12 query blocks of the fp32 kernels, causal and not."""
    from gonn_amd import hip
    B, H, S = 1, 2, 1536
    q, k, v, g = (randn((B * H, S, D), 4500 + D + int(causal) + i) for i in range(4))
    dev = [torch.from_numpy(x).cuda() for x in (q, k, v, g)]
    say(f"bwd fp32 full rows S={S} D={D} causal={causal}")
    o, l = hip.attn_fwd(*dev[:3], causal=causal, mode="fp32")
    dq, dk, dv = hip.attn_bwd(*dev[:3], o, l, dev[3], causal=causal, mode="fp32")
    torch.cuda.synchronize()
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, causal=causal)
    assert_close(dq.cpu().numpy(), rq, "fp32", "dQ")
    assert_close(dk.cpu().numpy(), rk, "fp32", "dK")
    assert_close(dv.cpu().numpy(), rv, "fp32", "dV")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("shape", [(592, 3, True), (1200, 8, False), (2400, 3, True)],
                         ids=lambda s: f"{s[0]}x{s[1]}{'c' if s[2] else ''}")
def test_bwd_long_query_few_keys(D, shape):
    """Cross-attention with many queries and a handful of keys (Sq >> Sk):
    each dK and dV row sums about Sq products of order 1, so it reaches 17 to
    90 while single entries of the same row can sit near 0. The bf16 bar
    (2e-2 + 1e-2 |ref| per entry) is stated for the N(0,1) self-attention
    configs; here the rounding of the inputs alone breaks it: the fp64
    oracle on bf16-rounded operands (Q * scale * log2(e), K, V, dO, as the
    kernels read them) differs from the oracle on the inputs by up to 0.14
    in dK and dV.

    The same holds for fp32 sums: 2400 terms of order 1 leave about 4e-6 of
    a row's size (1.3e-4 on an entry of 33), past the fp32-mode 1e-4.
    So both bars are taken per row here (the row's largest |ref| in place of
    the entry's own |ref|). Checks, per case:
    - fp32 mode, the same inputs: every entry within
      1e-4 + 1e-5 * (largest |ref| of its row), so the kernels' blocking,
      causal limits and key tails are right at this shape;
    - bf16 mode against the oracle on the rounded operands (the kernels' own
      rounding: bf16 P and dS, fp32 sums): every entry within
      2e-2 + 1e-2 * (largest |ref| of its row);
    - bf16 mode against the oracle on the inputs: the worst entry at most
      twice the worst difference the input rounding alone makes, plus 2e-2.
    A query block left out of a dK or dV sum moves its rows by 64/Sq of
    their size (3% to 11% here) and fails the row bar."""
    from tests._util import bf16_round
    Sq, Sk, causal = shape
    BH = 4
    seed = 4700 + Sq + Sk + D
    q, g = (randn((BH, Sq, D), seed + i) for i in range(2))
    k, v = (randn((BH, Sk, D), seed + 2 + i) for i in range(2))
    sc = 1.0 / math.sqrt(D)
    say(f"bwd long-query few-key D={D} Sq={Sq} Sk={Sk} causal={causal}")
    def row_bar(got, ref, atol, rtol, what):
        err = np.abs(got.astype(np.float64) - ref)
        bound = atol + rtol * np.abs(ref).max(axis=-1, keepdims=True)
        worst = np.unravel_index(int(np.argmax(err - bound)), err.shape)
        say(f"[{what}] max_abs={err.max():.3e} row bar ok: {bool(np.all(err <= bound))}")
        assert np.all(err <= bound), (what, worst, got[worst], ref[worst])

    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, sc, causal)
    _, _, dq, dk, dv = _fwd_bwd(q, k, v, g, causal, "fp32")
    for got, ref, n in ((dq, rq, "dQ"), (dk, rk, "dK"), (dv, rv, "dV")):
        row_bar(got, ref, 1e-4, 1e-5, f"{n} fp32")
    c2 = np.float32(sc * math.log2(math.e))
    qr = bf16_round(q * c2).astype(np.float64) / np.float64(c2)
    bq, bk, bv = oracle.attn_bwd_autograd(qr, bf16_round(k), bf16_round(v), bf16_round(g),
                                          sc, causal)
    _, _, dq, dk, dv = _fwd_bwd(q, k, v, g, causal, "bf16")
    for got, ref, bref, n in ((dq, rq, bq, "dQ"), (dk, rk, bk, "dK"), (dv, rv, bv, "dV")):
        row_bar(got, bref, 2e-2, 1e-2, f"{n} bf16 vs rounded operands")
        inputs = np.abs(bref - ref).max()
        err = np.abs(got.astype(np.float64) - ref).max()
        say(f"[{n} bf16] vs inputs {err:.3e}, input rounding alone {inputs:.3e}")
        assert err <= 2 * inputs + 2e-2, n


def test_bwd_golden_fixtures_via_f64_entry():
    """The committed torch-fp64 fixtures (square cases) through the reference-
    named f64 entry points FlashAttnF64Fwd / FlashAttnF64Bwd (head dims below
    64 are zero-padded on the device), at the fp32-MFMA bar."""
    import os
    from gonn_amd import hip
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "attn_golden.npz"))
    names = sorted({f.split("/")[0] for f in z.files})
    ran = 0
    for n in names:
        BH, Sq, Sk, D, causal, H = (int(x) for x in z[n + "/meta"])
        if Sq != Sk or (n + "/kv_len") in z.files:
            continue
        say(f"golden bwd {n}")
        q, k, v, g = (z[n + "/" + x] for x in ("q", "k", "v", "dO"))
        scale = 1.0 / math.sqrt(D)
        O, L = hip.FlashAttnF64Fwd(q, k, v, BH, Sq, D, scale, bool(causal))
        assert_close(O.reshape(BH, Sq, D), z[n + "/O"], "fp32", f"{n} O")
        assert_close(L.reshape(BH, Sq), z[n + "/LSE"], "fp32", f"{n} LSE")
        dQ, dK, dV = hip.FlashAttnF64Bwd(q, k, v, O, L, g, BH, Sq, D, scale, bool(causal))
        for nm, got in (("dQ", dQ), ("dK", dK), ("dV", dV)):
            assert_close(got.reshape(BH, Sq, D), z[n + "/" + nm], "fp32", f"{n} {nm}")
        ran += 1
    assert ran >= 4


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_flashbwd_shape_via_f64_entry(causal):
    """The reference's flashbwd check shape (benchmark/flashbwd/main.go:40-95:
    BH=2, S=6, D=64, loss = sum(O * dO)) through FlashAttnF64Bwd, against the
    oracle's gradients (which pass that program's finite-difference check)."""
    from gonn_amd import hip
    rng = np.random.default_rng(1)
    BH, S, D = 2, 6, 64
    Q, K, V, dO = (rng.standard_normal(BH * S * D) for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    O, L = hip.FlashAttnF64Fwd(Q, K, V, BH, S, D, scale, causal)
    dQ, dK, dV = hip.FlashAttnF64Bwd(Q, K, V, O, L, dO, BH, S, D, scale, causal)
    shp = (BH, S, D)
    rq, rk, rv = oracle.attn_bwd_autograd(Q.reshape(shp), K.reshape(shp), V.reshape(shp),
                                          dO.reshape(shp), causal=causal)
    assert_close(dQ.reshape(shp), rq, "fp32", "dQ")
    assert_close(dK.reshape(shp), rk, "fp32", "dK")
    assert_close(dV.reshape(shp), rv, "fp32", "dV")


def _sample(S, n, seed):
    rng = np.random.default_rng(seed)
    fixed = [0, 1, 63, 64, 127, 128, S // 2, S - 129, S - 2, S - 1]
    return np.array(sorted(set(fixed) | set(rng.integers(0, S, n).tolist())), dtype=np.int32)


def test_c5_fwd_bwd_full_size():
    """C5: B=2 H=16 S=8192 D=128 causal, bf16 MFMA, forward + backward.

    The oracle runs the full fp64 forward (O, LSE checked on every row) and
    the closed-form backward on 48+ sampled query rows (dQ) and key rows (dK,
    dV). On
    the full output: sum_j dV_j = sum_i dO_i (rows of P sum to 1) and
    sum_j dK_j = 0 (sum_j dS_ij = 0), per (b,h) and column; two runs are
    bit-identical (no atomics)."""
    B, H, S, D = 2, 16, 8192, 128
    mode = "bf16"
    BH = B * H
    q, k, v, g = (randn((BH, S, D), 500 + i) for i in range(4))
    say("C5 run")
    o, l, dq, dk, dv = _fwd_bwd(q, k, v, g, True, mode)
    for x in (o, l, dq, dk, dv):
        assert np.all(np.isfinite(x))
    say("C5 oracle forward")
    ro, rl = oracle.attn_fwd(q, k, v, causal=True)
    assert_close(o, ro, mode, "C5 O")
    assert_close(l, rl, mode, "C5 LSE")
    rows = _sample(S, 48, 9)
    say("C5 oracle backward rows")
    rq, rk, rv = oracle.attn_bwd_rows(q, k, v, ro, rl, g, causal=True, qrows=rows, krows=rows)
    assert_close(dq[:, rows], rq[:, rows], mode, "C5 dQ")
    assert_close(dk[:, rows], rk[:, rows], mode, "C5 dK")
    assert_close(dv[:, rows], rv[:, rows], mode, "C5 dV")
    # Identities over the full output (fp64 sums of the fp32 results).
    # Error model of sum_j dV_j - sum_i dO_i = sum_i dO_i (sum_j P~_ij - 1):
    # the bf16 P~ and the LSE error (~1e-3, up to 7e-3 on the first rows)
    # give per-row deviations eps_i ~ 1.5e-3, so each of the 32 x 128 column
    # sums is ~N(0, sqrt(8192) * 1.5e-3 = 0.14); the largest of 4096 lands near
    # 0.5. atol 1.0 (~7 sigma) still flags any dropped or repeated key tile,
    # which moves a column sum by O(10).
    np.testing.assert_allclose(dv.astype(np.float64).sum(axis=1),
                               g.astype(np.float64).sum(axis=1), atol=1.0, rtol=1e-3)
    assert np.abs(dk.astype(np.float64).sum(axis=1)).max() < 0.5
    say("C5 determinism")
    _, _, dq2, dk2, dv2 = _fwd_bwd(q, k, v, g, True, mode)
    assert np.array_equal(dq2, dq) and np.array_equal(dk2, dk) and np.array_equal(dv2, dv)
