"""GPU parity of the KV-cache handle (gonn_hip_kvcache_*) and of
MultiHeadAttention.forward_incremental.

The reference has no KV cache; what pins the results is the attention it
computes without one:
  * incremental self-attention over a cache equals the causal rows of
    MultiHeadAttention.Forward over the whole sequence (top-left causal mask,
    nn/attention.go:185-196), checked against the fp64 oracle's mha_fwd;
  * attending a cache with per-sequence lengths equals ForwardMasked with a
    key-padding mask (nn/attention.go:305-341), checked against the oracle's
    attn_fwd with kv_len.
The cache stores bf16 K/V: fed the same bf16-rounded values the oracle bar is
the fp32 one (max-abs 1e-4); fed fp64 values (the MHA test) it is the bf16 bar.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_round, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _mha_params(E, seed):
    s = 1.0 / math.sqrt(E)
    p = {}
    for i, n in enumerate(("q", "k", "v", "o")):
        p["W" + n] = randn((E, E), seed + 2 * i).astype(np.float64) * s
        p["b" + n] = randn((E,), seed + 2 * i + 1).astype(np.float64) * 0.1
    return p


@pytest.mark.parametrize("E,H", [(256, 4), (256, 2)], ids=["D64", "D128"])
def test_incremental_mha_matches_causal_forward(E, H):
    from gonn_amd import nn
    B, T = 2, 24
    say(f"[kvcache] incremental MHA B={B} T={T} E={E} H={H}")
    p = _mha_params(E, 700 + H)
    x = randn((B, T, E), 710 + H).astype(np.float64)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    ref = oracle.mha_fwd(x, x, x, p, H, causal=True)
    with mha.new_cache(B, 32) as cache:
        y1 = mha.forward_incremental(x[:, :10], cache)
        y2 = mha.forward_incremental(x[:, 10:], cache)
        assert list(cache.lengths()) == [T, T]
    got = np.concatenate([y1, y2], axis=1)
    assert_close(got, ref, "bf16", f"incremental MHA D={E // H}")


@pytest.mark.parametrize("D", [64, 128])
def test_ragged_append_attend_matches_key_padding(D):
    from gonn_amd import hip
    B, H, Lmax = 3, 2, 200
    say(f"[kvcache] ragged append D={D}")
    k1 = bf16_round(randn((B, H, 70, D), 720 + D)).astype(np.float64)
    v1 = bf16_round(randn((B, H, 70, D), 721 + D)).astype(np.float64)
    k2 = bf16_round(randn((B, H, 50, D), 722 + D)).astype(np.float64)
    v2 = bf16_round(randn((B, H, 50, D), 723 + D)).astype(np.float64)
    q = bf16_round(randn((B, H, D), 724 + D)).astype(np.float64)
    c1, c2 = [70, 1, 0], [50, 0, 37]
    with hip.KVCache(B, H, Lmax, D) as cache:
        cache.append_f64(k1, v1, counts=c1)
        cache.append_f64(k2, v2, counts=c2)
        lens = [a + b for a, b in zip(c1, c2)]
        assert list(cache.lengths()) == lens
        got = cache.attend_f64(q)
        # the same positions laid out for the oracle: keys 0..len_b-1
        K = np.zeros((B, H, Lmax, D))
        V = np.zeros((B, H, Lmax, D))
        for b in range(B):
            K[b, :, :c1[b]] = k1[b, :, :c1[b]]
            V[b, :, :c1[b]] = v1[b, :, :c1[b]]
            K[b, :, c1[b]:lens[b]] = k2[b, :, :c2[b]]
            V[b, :, c1[b]:lens[b]] = v2[b, :, :c2[b]]
        valid = [b for b in range(B) if lens[b] > 0]
        O, _ = oracle.attn_fwd(q.reshape(B * H, 1, D), K.reshape(B * H, Lmax, D),
                               V.reshape(B * H, Lmax, D), 1.0 / math.sqrt(D), False,
                               kv_len=lens, H=H)
        ref = O.reshape(B, H, D)
        assert_close(got[valid], ref[valid], "fp32", f"ragged append D={D}")
        # overflow is rejected and writes nothing
        with pytest.raises(hip.GonnHipError) as ei:
            cache.append_f64(np.zeros((B, H, 100, D)), np.zeros((B, H, 100, D)))
        assert ei.value.code == -1
        assert list(cache.lengths()) == lens
        assert_close(cache.attend_f64(q)[valid], ref[valid], "fp32", "after rejected append")
        cache.reset()
        assert list(cache.lengths()) == [0, 0, 0]
        assert np.all(cache.attend_f64(q) == 0.0)


@pytest.mark.parametrize("src", ["bf16", "f32"])
def test_device_append_matches_decode_on_filled_cache(src):
    from gonn_amd import hip
    B, H, Lmax, D = 4, 8, 256, 128
    say(f"[kvcache] device append src={src}")
    dt = torch.bfloat16 if src == "bf16" else torch.float32
    k = torch.from_numpy(randn((B, H, 96, D), 730)).cuda().to(dt)
    v = torch.from_numpy(randn((B, H, 96, D), 731)).cuda().to(dt)
    q = torch.from_numpy(randn((B, H, D), 732)).cuda()
    counts = [96, 40, 1, 77]
    with hip.KVCache(B, H, Lmax, D) as cache:
        cache.append(k[:, :, :50].contiguous(), v[:, :, :50].contiguous(),
                     counts=[min(c, 50) for c in counts])
        rest = [max(c - 50, 0) for c in counts]
        cache.append(k[:, :, 50:].contiguous(), v[:, :, 50:].contiguous(), counts=rest)
        assert list(cache.lengths()) == counts
        got = cache.attend(q)
        kc = torch.zeros((B, H, Lmax, D), dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros_like(kc)
        for b, c in enumerate(counts):
            kc[b, :, :c] = k[b, :, :c].to(torch.bfloat16)
            vc[b, :, :c] = v[b, :, :c].to(torch.bfloat16)
        kl = torch.tensor(counts, dtype=torch.int32, device="cuda")
        ref = hip.attn_decode(q, kc, vc, kl)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (got - ref).abs().max().item()
