"""GPU parity of the flash forward against the fp64 oracle (through the C ABI).

Configs: small ragged shapes for both modes, D in {64, 128}, causal and not,
Sq != Sk (top-left causal); BASELINE configs C2 (encoder) and C3 (causal
prefill) at full size on sampled query rows, plus size-independent properties
at full size (causal invariance, Q = 0 prefix means, determinism); bfloat16
inputs against their float32 widening (bit-identical outputs).
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import TOL, assert_close, bf16_round, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _run(q, k, v, causal, mode, scale=None):
    from gonn_amd import hip
    o, l = hip.attn_fwd(_dev(q), _dev(k), _dev(v), causal=causal, mode=mode, scale=scale)
    torch.cuda.synchronize()
    return o.cpu().numpy(), l.cpu().numpy()


def test_mfma_layout_selftest():
    from gonn_amd import hip
    assert hip.Available(), "no gfx950 device visible"
    assert hip.SelftestMFMA() == 0


SMALL = [  # (BH, Sq, Sk)
    (1, 1, 1), (2, 7, 7), (3, 37, 37), (2, 64, 64), (2, 128, 128), (2, 129, 129),
    (1, 200, 200), (2, 130, 300), (2, 300, 129), (1, 1, 257),
]


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "x".join(map(str, s)))
def test_fwd_small(mode, D, causal, shape):
    BH, Sq, Sk = shape
    seed = 1000 * BH + 7 * Sq + Sk + D + int(causal)
    q, k, v = randn((BH, Sq, D), seed), randn((BH, Sk, D), seed + 1), randn((BH, Sk, D), seed + 2)
    say(f"fwd_small mode={mode} D={D} causal={causal} shape={shape}")
    o, l = _run(q, k, v, causal, mode)
    ro, rl = oracle.attn_fwd(q, k, v, causal=causal)
    assert_close(o, ro, mode, "O")
    assert_close(l, rl, mode, "LSE")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_fwd_scale_variants(mode):
    """Negative and zero scale follow softmax(scale*QK^T) like the reference."""
    BH, S, D = 2, 96, 64
    q, k, v = randn((BH, S, D), 5), randn((BH, S, D), 6), randn((BH, S, D), 7)
    for scale in (-0.2, 0.0, 0.05):
        o, l = _run(q, k, v, True, mode, scale=scale)
        ro, rl = oracle.attn_fwd(q, k, v, scale=scale, causal=True)
        assert_close(o, ro, mode, f"O scale={scale}")
        assert_close(l, rl, mode, f"LSE scale={scale}")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_c2_encoder_full_size(mode):
    """C2: B=8 H=12 S=1024 D=64 non-causal, every row against the oracle."""
    B, H, S, D = 8, 12, 1024, 64
    q = randn((B * H, S, D), 21)
    k = randn((B * H, S, D), 22)
    v = randn((B * H, S, D), 23)
    say(f"C2 mode={mode}")
    o, l = _run(q, k, v, False, mode)
    ro, rl = oracle.attn_fwd(q, k, v, causal=False)
    assert_close(o, ro, mode, "C2 O")
    assert_close(l, rl, mode, "C2 LSE")


def test_c3_prefill_full_size():
    """C3: B=4 H=32 S=4096 D=128 causal, bf16 MFMA; every row against the
    oracle, plus size-independent properties on the full output."""
    B, H, S, D = 4, 32, 4096, 128
    mode = "bf16"
    q = randn((B * H, S, D), 31)
    k = randn((B * H, S, D), 32)
    v = randn((B * H, S, D), 33)
    say("C3 parity")
    o, l = _run(q, k, v, True, mode)
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(l))
    say("C3 oracle forward (every row)")
    ro, rl = oracle.attn_fwd(q, k, v, causal=True)
    assert_close(o, ro, mode, "C3 O")
    assert_close(l, rl, mode, "C3 LSE")
    del ro, rl
    # Causal invariance: changing keys/values at positions > p leaves rows <= p
    # bit-identical (masked keys carry exactly zero weight).
    p = 2500
    k2, v2 = k.copy(), v.copy()
    k2[:, p + 1:] = k2[:, p + 1:] * -3.0 + 1.0
    v2[:, p + 1:] = v2[:, p + 1:] + 5.0
    o2, l2 = _run(q, k2, v2, True, mode)
    assert np.array_equal(o2[:, :p + 1], o[:, :p + 1])
    assert np.array_equal(l2[:, :p + 1], l[:, :p + 1])
    assert not np.array_equal(o2[:, p + 1:], o[:, p + 1:])
    # Determinism: same inputs, bit-identical outputs.
    o3, l3 = _run(q, k, v, True, mode)
    assert np.array_equal(o3, o) and np.array_equal(l3, l)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_zero_query_gives_prefix_mean(mode):
    """Q = 0: every unmasked weight is equal, so O_i is the mean of V rows 0..i
    (of the bf16-rounded V in bf16 mode) and LSE_i = ln(i+1)."""
    BH, S, D = 4, 1000, 128
    q = np.zeros((BH, S, D), np.float32)
    k, v = randn((BH, S, D), 41), randn((BH, S, D), 42)
    o, l = _run(q, k, v, True, mode)
    vv = (bf16_round(v) if mode == "bf16" else v).astype(np.float64)
    ref = np.cumsum(vv, axis=1) / np.arange(1, S + 1)[None, :, None]
    np.testing.assert_allclose(o, ref, atol=2e-5, rtol=0)
    np.testing.assert_allclose(l, np.broadcast_to(np.log(np.arange(1, S + 1)), (BH, S)),
                               atol=2e-5, rtol=0)


def test_ref_shape_refattn_protocol():
    """The reference's own fused-vs-refAttn protocol (benchmark/flashattn/
    main.go:103-123): BH=3, S=12, d=8, both mask settings, through the f64
    FlashAttnF64 entry point; d=8 is zero-padded to 64 on the device."""
    from gonn_amd import hip
    for causal in (False, True):
        BH, S, d = 3, 12, 8
        rng = np.random.default_rng(7)
        Q, K, V = (rng.standard_normal(BH * S * d) for _ in range(3))
        O = np.zeros(BH * S * d)
        scale = 1.0 / math.sqrt(d)
        hip.FlashAttnF64(Q, K, V, O, BH, S, d, scale, causal)
        ref = oracle.ref_attn(Q.reshape(BH, S, d), K.reshape(BH, S, d), V.reshape(BH, S, d),
                              scale, causal)
        # the fused fp64 kernel met 1e-9; fp32-MFMA meets the fp32 bar
        assert_close(O.reshape(BH, S, d), ref, "fp32", f"refAttn causal={causal}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 64, 64), (2, 129, 129), (1, 200, 200), (2, 130, 300),
                                   (2, 1000, 1000)], ids=lambda s: "x".join(map(str, s)))
def test_fwd_bf16_inputs_match_f32_inputs(D, causal, shape):
    """bf16-mode forward on bfloat16 Q/K/V against the same call on their
    float32 widening: the kernels round the same products (Q * sign * c2 and
    the packed K/V) to bf16, so O and LSE must agree bit for bit; the float32
    path is the one pinned to the oracle above. Covers the QT = bf16 kernel
    instantiations and the bf16 pack, with ragged and multi-tile blocks."""
    from gonn_amd import hip
    BH, Sq, Sk = shape
    say(f"[fwd bf16 inputs] D={D} causal={causal} shape={shape}")
    g = torch.Generator(device="cuda").manual_seed(Sq * 31 + Sk + D + int(causal))
    qb, kb, vb = (torch.randn((BH, S, D), generator=g, device="cuda").to(torch.bfloat16)
                  for S in (Sq, Sk, Sk))
    o16, l16 = hip.attn_fwd(qb, kb, vb, causal=causal, mode="bf16")
    o32, l32 = hip.attn_fwd(qb.float(), kb.float(), vb.float(), causal=causal, mode="bf16")
    torch.cuda.synchronize()
    assert torch.equal(o16, o32), float((o16 - o32).abs().max())
    assert torch.equal(l16, l32), float((l16 - l32).abs().max())


def test_fwd_bf16_inputs_masked_and_kv_len():
    """The same equality through the additive-mask (D = 64) and kv_len paths."""
    from gonn_amd import hip
    B, H, S, D = 2, 3, 150, 64
    g = torch.Generator(device="cuda").manual_seed(77)
    qb, kb, vb = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16)
                  for _ in range(3))
    mask = torch.randn((B, S, S), generator=g, device="cuda")
    kv_len = torch.tensor([150, 97], dtype=torch.int32, device="cuda")
    for kw in ({"attn_mask": mask}, {"kv_len": kv_len, "causal": True}):
        o16, l16 = hip.attn_fwd(qb, kb, vb, mode="bf16", **kw)
        o32, l32 = hip.attn_fwd(qb.float(), kb.float(), vb.float(), mode="bf16", **kw)
        torch.cuda.synchronize()
        assert torch.equal(o16, o32), (list(kw), float((o16 - o32).abs().max()))
        assert torch.equal(l16, l32), list(kw)
