"""GPU parity of the causal multi-token cache attend (gonn_hip_kvcache_attend_causal)
and of the device-resident incremental MHA (gonn_hip_mha_forward_incremental_dev).

Both are new relative to the reference, which has no KV cache. What pins them
is the attention it computes over whole sequences:
  * T new queries whose K/V are the last T cached positions: query t of
    sequence b attends positions [0, len_b - T + t], the top-left causal
    mask of nn/attention.go:185-196 over the whole sequence; checked per
    query against the fp64 oracle's attn_fwd on exactly those positions;
  * the resident incremental layer equals the causal rows of
    MultiHeadAttention.Forward (nn/attention.go:107-148) over the whole
    sequence, checked against the oracle's mha_fwd.
The cache stores bf16 K/V: fed bf16-rounded values the bar is the fp32 one;
fed fp64 values (the MHA tests) it is the bf16 bar.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_round, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _filled_cache(hip, B, H, Lmax, D, lens, seed):
    K = bf16_round(randn((B, H, Lmax, D), seed)).astype(np.float64)
    V = bf16_round(randn((B, H, Lmax, D), seed + 1)).astype(np.float64)
    cache = hip.KVCache(B, H, Lmax, D)
    cache.append_f64(K[:, :, :max(lens)], V[:, :, :max(lens)], counts=lens)
    return cache, K, V


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("T", [1, 3, 4, 9])
def test_attend_causal_matches_per_query_oracle(D, T):
    from gonn_amd import hip
    B, H, Lmax = 3, 2, 320
    lens = [T, 150 + T, 311]
    say(f"[kvcache-causal] D={D} T={T} lens={lens}")
    cache, K, V = _filled_cache(hip, B, H, Lmax, D, lens, 800 + D + T)
    with cache:
        q = bf16_round(randn((B, H, T, D), 810 + T))
        got = cache.attend_causal(torch.from_numpy(q).cuda()).cpu().numpy()
        ref = np.zeros((B, H, T, D))
        for b in range(B):
            for t in range(T):
                lim = lens[b] - T + t + 1
                o, _ = oracle.attn_fwd(q[b, :, t:t + 1].astype(np.float64), K[b, :, :lim],
                                       V[b, :, :lim], 1.0 / math.sqrt(D), False)
                ref[b, :, t] = o[:, 0]
        assert_close(got, ref, "fp32", f"attend_causal D={D} T={T}")
        if T == 1:
            one = cache.attend(torch.from_numpy(q[:, :, 0]).cuda()).cpu().numpy()
            assert_close(got[:, :, 0], one, "fp32", "attend_causal T=1 vs attend")


def test_attend_causal_signed_scale_and_long_range():
    from gonn_amd import hip
    B, H, Lmax, D, T = 2, 4, 5000, 128, 5
    lens = [4999, 2048]
    say(f"[kvcache-causal] long range lens={lens}")
    cache, K, V = _filled_cache(hip, B, H, Lmax, D, lens, 830)
    with cache:
        q = bf16_round(randn((B, H, T, D), 831))
        for scale in (-0.05, 0.2):
            got = cache.attend_causal(torch.from_numpy(q).cuda(), scale=scale).cpu().numpy()
            for b in range(B):
                for t in (0, T - 1):
                    lim = lens[b] - T + t + 1
                    o, _ = oracle.attn_fwd(q[b, :, t:t + 1].astype(np.float64), K[b, :, :lim],
                                           V[b, :, :lim], scale, False)
                    assert_close(got[b, :, t], o[:, 0], "fp32", f"long range b={b} t={t} s={scale}")


def test_attend_causal_rejects_short_cache_and_workspace():
    from gonn_amd import hip
    B, H, Lmax, D = 2, 2, 64, 64
    with hip.KVCache(B, H, Lmax, D) as cache:
        z = np.zeros((B, H, 3, D))
        cache.append_f64(z, z, counts=[3, 2])
        q = torch.zeros((B, H, 3, D), device="cuda")
        with pytest.raises(hip.GonnHipError) as ei:
            cache.attend_causal(q)  # sequence 1 holds 2 < T positions
        assert ei.value.code == -1
        small = torch.empty(16, dtype=torch.uint8, device="cuda")
        with pytest.raises(hip.GonnHipError) as ei:
            cache.attend_causal(q[:, :, :2].contiguous(), ws=small)
        assert ei.value.code == -3


def _mha(E, H, seed):
    from gonn_amd import nn
    s = 1.0 / math.sqrt(E)
    p = {}
    for i, n in enumerate(("q", "k", "v", "o")):
        p["W" + n] = randn((E, E), seed + 2 * i).astype(np.float64) * s
        p["b" + n] = randn((E,), seed + 2 * i + 1).astype(np.float64) * 0.1
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    return mha, p


@pytest.mark.parametrize("E,H", [(256, 4), (256, 2), (64, 2)], ids=["D64", "D128", "D32"])
def test_resident_incremental_matches_causal_forward(E, H):
    B, T = 3, 30
    say(f"[kvcache-causal] resident incremental E={E} H={H}")
    mha, p = _mha(E, H, 840 + E + H)
    x = randn((B, T, E), 850 + H).astype(np.float64)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=True)
    with mha.to_device() as res, res.new_cache(B, 40) as cache:
        chunks = [(0, 11), (11, 12), (12, 17), (17, 30)]
        got = np.concatenate([res.forward_incremental(x[:, a:b], cache) for a, b in chunks], axis=1)
        assert list(cache.lengths()) == [T] * B
    assert_close(got, ref, "bf16", f"resident incremental D={E // H}")


def test_resident_incremental_device_buffers_and_failure_keeps_lengths():
    from gonn_amd import hip
    E, H, B = 256, 2, 2
    mha, p = _mha(E, H, 870)
    x = randn((B, 8, E), 871).astype(np.float64)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=True)
    with mha.to_device() as res, res.new_cache(B, 8) as cache:
        dev = res.dev
        xd = torch.from_numpy(x).cuda()
        ws = torch.empty(dev.incremental_workspace_bytes(cache, 4), dtype=torch.uint8,
                         device="cuda")
        y1 = dev.forward_incremental_dev(xd[:, :4].contiguous(), cache, ws=ws)
        y2 = dev.forward_incremental_dev(xd[:, 4:].contiguous(), cache, ws=ws)
        torch.cuda.synchronize()
        got = torch.cat([y1, y2], dim=1).cpu().numpy()
        assert_close(got, ref, "bf16", "resident incremental, device buffers")
        # the cache is full: one more position is rejected and changes nothing
        with pytest.raises(hip.GonnHipError) as ei:
            dev.forward_incremental_dev(xd[:, :1].contiguous(), cache)
        assert ei.value.code == -1
        assert list(cache.lengths()) == [8, 8]
    # a cache of the wrong head dim does not fit the layer
    with mha.to_device() as res, hip.KVCache(B, H, 8, 64) as wrong:
        with pytest.raises(ValueError):
            res.dev.forward_incremental_dev(torch.zeros((B, 1, E), dtype=torch.float64,
                                                        device="cuda"), wrong)
