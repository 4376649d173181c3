"""GPU parity of the f64 entry points in their exact mode (GONN_ATTN_FP64):
fp64 kernels throughout, held to the reference's own fp64 gates.

GoNN's CUDA seam computes in fp64 (backend/cuda/gonn_cuda.cu:302-529), and
its checking programs gate the fused path at that precision:
- benchmark/flashattn/main.go:103-123: FlashAttnF64 against refAttn, max abs
  diff <= 1e-9 (BH=3, S=12, d=8, both mask settings);
- benchmark/mha/main.go:64: MultiHeadAttention.ForwardFused against
  Forward, <= 1e-9;
- benchmark/flashbwd/main.go:40-95: FlashAttnF64Bwd against central
  differences of sum(O * dO) through FlashAttnF64Fwd, eps 1e-6, relative
  error <= 1e-4 (BH=2, S=6, D=64, indices 0, 1, 64, 130, 200, n-1).
These tests run exactly those protocols through the library, plus the
torch-fp64 golden fixtures, key padding, additive masks and Sq != Sk
against the fp64 oracle at 1e-11.
"""
import math
import os

import numpy as np
import pytest

import oracle
from tests._util import say

pytestmark = pytest.mark.gpu

F64_ATOL = 1e-11  # fp64 kernels against an fp64 CPU evaluation


@pytest.fixture
def f64_mode():
    from gonn_amd import hip
    prev = hip.AttnMode()
    hip.SetAttnMode("f64")
    try:
        yield hip
    finally:
        hip.SetAttnMode(prev)


def _close(got, ref, what, atol=F64_ATOL):
    err = float(np.max(np.abs(np.asarray(got, dtype=np.float64) - ref)))
    print(f"[{what}] f64 max_abs={err:.3e} (bar {atol:g})", flush=True)
    assert np.all(np.isfinite(got)), what
    assert err <= atol, (what, err)


@pytest.mark.parametrize("causal", [False, True])
def test_refattn_protocol_at_the_reference_gate(f64_mode, causal):
    """benchmark/flashattn: BH=3, S=12, d=8 against refAttn at <= 1e-9."""
    hip = f64_mode
    BH, S, d = 3, 12, 8
    rng = np.random.default_rng(7)
    Q, K, V = (rng.standard_normal(BH * S * d) for _ in range(3))
    O = np.zeros(BH * S * d)
    scale = 1.0 / math.sqrt(d)
    say(f"f64 refAttn causal={causal}")
    hip.FlashAttnF64(Q, K, V, O, BH, S, d, scale, causal)
    ref = oracle.ref_attn(Q.reshape(BH, S, d), K.reshape(BH, S, d), V.reshape(BH, S, d), scale,
                          causal)
    _close(O.reshape(BH, S, d), ref, f"refAttn causal={causal}", atol=1e-9)
    _close(O.reshape(BH, S, d), ref, f"refAttn causal={causal}")


@pytest.mark.parametrize("causal", [False, True])
def test_flashbwd_gradcheck_protocol(f64_mode, causal):
    """benchmark/flashbwd: central differences of sum(O * dO) through the
    library's own forward against its backward, eps 1e-6, rel <= 1e-4 (the
    fp32 and bf16 modes cannot pass this: their forward's rounding swamps
    a 1e-6 step)."""
    hip = f64_mode
    BH, S, D = 2, 6, 64
    n = BH * S * D
    scale = 1.0 / math.sqrt(D)
    rng = np.random.default_rng(11 + int(causal))
    Q, K, V, dO = (rng.uniform(-1, 1, n) for _ in range(4))
    say(f"f64 flashbwd gradcheck causal={causal}")
    O, L = hip.FlashAttnF64Fwd(Q, K, V, BH, S, D, scale, causal)
    dQ, dK, dV = hip.FlashAttnF64Bwd(Q, K, V, O, L, dO, BH, S, D, scale, causal)
    eps = 1e-6

    def num_grad(x, idx):
        save = x[idx]
        x[idx] = save + eps
        lp = float(np.sum(hip.FlashAttnF64Fwd(Q, K, V, BH, S, D, scale, causal)[0] * dO))
        x[idx] = save - eps
        lm = float(np.sum(hip.FlashAttnF64Fwd(Q, K, V, BH, S, D, scale, causal)[0] * dO))
        x[idx] = save
        return (lp - lm) / (2 * eps)

    worst = 0.0
    for name, ag, x in (("dQ", dQ, Q), ("dK", dK, K), ("dV", dV, V)):
        for idx in (0, 1, 64, 130, 200, n - 1):
            ng = num_grad(x, idx)
            a = float(np.ravel(ag)[idx])
            rel = abs(ng - a) / (abs(ng) + abs(a) + 1e-9)
            worst = max(worst, rel)
            assert rel <= 1e-4, (name, idx, a, ng, rel)
    print(f"[flashbwd causal={causal}] maxRelErr={worst:.2e}", flush=True)


def test_golden_fixtures(f64_mode):
    """The committed torch-fp64 fixtures through FlashAttnF64Fwd / Bwd."""
    hip = f64_mode
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "attn_golden.npz"))
    names = sorted({f.split("/")[0] for f in z.files})
    ran = 0
    for nm in names:
        BH, Sq, Sk, D, causal, H = (int(x) for x in z[nm + "/meta"])
        if Sq != Sk or (nm + "/kv_len") in z.files:
            continue
        say(f"f64 golden {nm}")
        q, k, v, g = (z[nm + "/" + x] for x in ("q", "k", "v", "dO"))
        scale = 1.0 / math.sqrt(D)
        O, L = hip.FlashAttnF64Fwd(q, k, v, BH, Sq, D, scale, bool(causal))
        _close(O.reshape(BH, Sq, D), z[nm + "/O"], f"{nm} O")
        _close(L.reshape(BH, Sq), z[nm + "/LSE"], f"{nm} LSE")
        dQ, dK, dV = hip.FlashAttnF64Bwd(q, k, v, O, L, g, BH, Sq, D, scale, bool(causal))
        for x, got in (("dQ", dQ), ("dK", dK), ("dV", dV)):
            _close(got.reshape(BH, Sq, D), z[nm + "/" + x], f"{nm} {x}")
        ran += 1
    assert ran >= 4


@pytest.mark.parametrize("d", [8, 64, 100, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_masked_cross_kv_len(f64_mode, d, causal):
    """Key padding, an additive (B, H, Sq, Sk) mask with blocked keys, and
    Sq != Sk in both directions, forward and backward, against the oracle."""
    hip = f64_mode
    from tests.test_gpu_masked import _mask_of
    B, H = 2, 2
    for Sq, Sk in ((33, 90), (70, 41)):
        lens = np.array([Sk, max(Sk // 3, 1)], dtype=np.int32)
        m, _ = _mask_of("BHTqTk4", B, H, Sq, Sk, 930 + d + Sq)
        rng = np.random.default_rng(940 + d + Sq + int(causal))
        q = rng.standard_normal((B * H, Sq, d))
        k = rng.standard_normal((B * H, Sk, d))
        v = rng.standard_normal((B * H, Sk, d))
        g = rng.standard_normal((B * H, Sq, d))
        scale = 1.0 / math.sqrt(d)
        say(f"f64 masked d={d} causal={causal} Sq={Sq} Sk={Sk}")
        O, L = hip.FlashAttnF64Ex(q, k, v, B, H, Sq, Sk, d, scale, causal, kv_len=lens, lse=True,
                                  attn_mask=m)
        ro, rl = oracle.attn_fwd(q, k, v, scale, causal, kv_len=lens, H=H, attn_mask=m)
        live = np.isfinite(rl)
        _close(O.reshape(ro.shape), ro, "O")
        assert np.array_equal(np.isfinite(L.reshape(rl.shape)), live)
        _close(L.reshape(rl.shape)[live], rl[live], "LSE")
        dQ, dK, dV = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, B, H, Sq, d, scale, causal,
                                           kv_len=lens, attn_mask=m, Sk=Sk)
        rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, scale=scale, causal=causal,
                                              kv_len=lens, H=H, attn_mask=m)
        for x, got, ref in (("dQ", dQ, rq), ("dK", dK, rk), ("dV", dV, rv)):
            _close(np.reshape(got, ref.shape), ref, x)


@pytest.mark.parametrize("kernels", ["mfma", "valu"])
@pytest.mark.parametrize("d", [64, 100, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_many_blocks_both_kernel_families(f64_mode, monkeypatch, kernels, d, causal):
    """Rows spanning several 64-row blocks and LDS stages, a ragged last
    block and key padding, through the MFMA kernels (default) and the team
    kernels (GONN_HIP_F64_FWD / GONN_HIP_F64_BWD = "valu"), forward and
    backward, against the oracle at the fp64 bar."""
    hip = f64_mode
    if kernels == "valu":
        monkeypatch.setenv("GONN_HIP_F64_FWD", "valu")
        monkeypatch.setenv("GONN_HIP_F64_BWD", "valu")
    B, H = 2, 2
    for Sq, Sk in ((333, 333), (150, 397)):
        lens = np.array([Sk, Sk // 2 + 7], dtype=np.int32)
        rng = np.random.default_rng(960 + d + Sq + int(causal))
        q, k, v, g = (rng.standard_normal((B * H, n, d)) for n in (Sq, Sk, Sk, Sq))
        scale = 1.0 / math.sqrt(d)
        say(f"f64 {kernels} d={d} causal={causal} Sq={Sq} Sk={Sk}")
        O, L = hip.FlashAttnF64Ex(q, k, v, B, H, Sq, Sk, d, scale, causal, kv_len=lens, lse=True)
        ro, rl = oracle.attn_fwd(q, k, v, scale, causal, kv_len=lens, H=H)
        _close(O.reshape(ro.shape), ro, "O")
        live = np.isfinite(rl)
        assert np.array_equal(np.isfinite(L.reshape(rl.shape)), live)
        _close(L.reshape(rl.shape)[live], rl[live], "LSE")
        dQ, dK, dV = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, B, H, Sq, d, scale, causal,
                                           kv_len=lens, Sk=Sk)
        rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, scale=scale, causal=causal,
                                              kv_len=lens, H=H)
        for x, got, ref in (("dQ", dQ, rq), ("dK", dK, rk), ("dV", dV, rv)):
            _close(np.reshape(got, ref.shape), ref, x)


@pytest.mark.parametrize("shape", [(64, 512), (32, 1024), (16, 2048)],
                         ids=lambda s: f"BH{s[0]}xS{s[1]}")
def test_causal_split_published_shapes(f64_mode, monkeypatch, shape):
    """GoNN's published causal shapes (benchmark/results/gonn_flash.json,
    d = 64). From 16 q-blocks of 64 rows on (S >= 961), the MFMA forward
    splits the key range of the later half of the q-blocks over two
    workgroups, whose partials (m, l, O) a combine kernel merges; it
    must equal the team kernel (GONN_HIP_F64_FWD=valu, no split, its own
    summation order) at the fp64 bar on every row, and the oracle on
    sampled rows."""
    hip = f64_mode
    BH, S = shape
    d = 64
    rng = np.random.default_rng(990 + S)
    q, k, v = (rng.standard_normal((BH, S, d)) for _ in range(3))
    scale = 1.0 / math.sqrt(d)
    say(f"f64 causal split BH={BH} S={S}")
    O, L = hip.FlashAttnF64Ex(q, k, v, BH, 1, S, S, d, scale, True, lse=True)
    monkeypatch.setenv("GONN_HIP_F64_FWD", "valu")
    Ov, Lv = hip.FlashAttnF64Ex(q, k, v, BH, 1, S, S, d, scale, True, lse=True)
    monkeypatch.delenv("GONN_HIP_F64_FWD")
    _close(O, Ov, "O split vs team kernel")
    _close(L, Lv, "LSE split vs team kernel")
    rows = np.array(sorted({0, 1, 63, 64, S // 2 - 1, S // 2, S - 65, S - 64, S - 1}),
                    dtype=np.int32)
    ro, rl = oracle.attn_fwd(q, k, v, scale, True, rows=rows)
    _close(O.reshape(BH, S, d)[:, rows], ro[:, rows], "O sampled rows")
    _close(L.reshape(BH, S)[:, rows], rl[:, rows], "LSE sampled rows")
    # the backward's split (dQ: the later q-blocks' key ranges; dK/dV: the
    # first key blocks' query ranges) against the team kernels
    g = rng.standard_normal((BH, S, d))
    got = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, BH, 1, S, d, scale, True)
    monkeypatch.setenv("GONN_HIP_F64_BWD", "valu")
    ref = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, BH, 1, S, d, scale, True)
    monkeypatch.delenv("GONN_HIP_F64_BWD")
    for x, a, b in zip(("dQ", "dK", "dV"), got, ref):
        _close(a, b, f"{x} split vs team kernels")


def test_causal_split_mask_kv_len(f64_mode):
    """The split causal forward and backward (16 q-blocks and key blocks at
    S = 1000) with key padding (one sequence ending inside a split q-block's
    first half) and an additive mask with blocked keys, against the oracle
    on every row."""
    hip = f64_mode
    from tests.test_gpu_masked import _mask_of
    B, H, S, d = 2, 2, 1000, 64
    lens = np.array([S, 545], dtype=np.int32)
    m, _ = _mask_of("BHTqTk4", B, H, S, S, 995)
    rng = np.random.default_rng(996)
    q, k, v = (rng.standard_normal((B * H, S, d)) for _ in range(3))
    scale = 1.0 / math.sqrt(d)
    say("f64 causal split, mask + kv_len")
    O, L = hip.FlashAttnF64Ex(q, k, v, B, H, S, S, d, scale, True, kv_len=lens, lse=True,
                              attn_mask=m)
    ro, rl = oracle.attn_fwd(q, k, v, scale, True, kv_len=lens, H=H, attn_mask=m)
    _close(O.reshape(ro.shape), ro, "O")
    live = np.isfinite(rl)
    assert np.array_equal(np.isfinite(L.reshape(rl.shape)), live)
    _close(L.reshape(rl.shape)[live], rl[live], "LSE")
    g = rng.standard_normal((B * H, S, d))
    dQ, dK, dV = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, B, H, S, d, scale, True, kv_len=lens,
                                       attn_mask=m)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, scale=scale, causal=True, kv_len=lens,
                                          H=H, attn_mask=m)
    for x, got, ref in (("dQ", dQ, rq), ("dK", dK, rk), ("dV", dV, rv)):
        _close(np.reshape(got, ref.shape), ref, x)


@pytest.mark.parametrize("d,Sq,Sk", [(128, 1030, 1030), (40, 1100, 1040), (100, 1000, 1500)],
                         ids=lambda x: str(x))
def test_causal_split_head_dims_and_cross(f64_mode, d, Sq, Sk):
    """The causal splits at other head widths (d = 40 runs the 64-wide
    kernels, 100 and 128 the 128-wide ones, with their own LDS stage) and
    with Sq != Sk (top-left causal: with Sq > Sk the later q-blocks all see
    every key; with Sq < Sk the last key blocks see no query). Every
    q-block count and key-block count here is at least 16, so the forward
    and both backward kernels run split; every row against the oracle."""
    hip = f64_mode
    B, H = 1, 2
    rng = np.random.default_rng(997 + d + Sq + Sk)
    q, k, v, g = (rng.standard_normal((B * H, n, d)) for n in (Sq, Sk, Sk, Sq))
    scale = 1.0 / math.sqrt(d)
    say(f"f64 causal split d={d} Sq={Sq} Sk={Sk}")
    O, L = hip.FlashAttnF64Ex(q, k, v, B, H, Sq, Sk, d, scale, True, lse=True)
    ro, rl = oracle.attn_fwd(q, k, v, scale, True)
    _close(O.reshape(ro.shape), ro, "O")
    _close(L.reshape(rl.shape), rl, "LSE")
    dQ, dK, dV = hip.FlashAttnF64BwdEx(q, k, v, O, L, g, B, H, Sq, d, scale, True, Sk=Sk)
    rq, rk, rv = oracle.attn_bwd_autograd(q, k, v, g, scale=scale, causal=True)
    for x, got, ref in (("dQ", dQ, rq), ("dK", dK, rk), ("dV", dV, rv)):
        _close(np.reshape(got, ref.shape), ref, x)


def test_mha_fused_protocol(f64_mode):
    """benchmark/mha: ForwardFused against the unfused Forward at <= 1e-9
    (the oracle's op sequence stands in for GoNN's CPU Forward)."""
    from gonn_amd import nn
    from tests.test_gpu_masked import _params
    B, T, E, H = 2, 16, 64, 2
    p = _params(E, 950)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    x = np.random.default_rng(951).standard_normal((B, T, E))
    for causal in (False, True):
        say(f"f64 mha causal={causal}")
        got = mha.forward_fused(x, x, x, causal)
        ref = oracle.mha_fwd(x, x, x, p, H, causal=causal)
        _close(got, ref, f"ForwardFused causal={causal}", atol=1e-9)


def test_bench_entry_times_the_fp64_kernel(f64_mode):
    hip = f64_mode
    ms = hip.BenchFlashAttnF64(4, 256, 64, 3, True)
    assert ms > 0.0, ms
