"""GPU parity of the split-KV decode against the oracle's key-padding path.

The oracle is ForwardMasked with WithKeyPaddingMask (nn/attention.go:305-341)
restated in attn_oracle.c; the kernel reads bf16 caches, so the oracle is fed
the same bf16-rounded values and the bar is the fp32 one (max-abs 1e-4).
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_round, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _case(B, H, Lmax, D, lens, seed, q_bf16=True):
    q = bf16_round(randn((B, H, D), seed))
    kc = bf16_round(randn((B, H, Lmax, D), seed + 1))
    vc = bf16_round(randn((B, H, Lmax, D), seed + 2))
    lens = np.asarray(lens, dtype=np.int32)
    qd = torch.from_numpy(q).cuda()
    qd = qd.to(torch.bfloat16) if q_bf16 else qd
    dev = dict(q=qd,
               kc=torch.from_numpy(kc).cuda().to(torch.bfloat16),
               vc=torch.from_numpy(vc).cuda().to(torch.bfloat16),
               kv_len=torch.from_numpy(lens).cuda())
    return q, kc, vc, lens, dev


def _run(dev, split_keys=0, scale=None):
    from gonn_amd import hip
    o = hip.attn_decode(dev["q"], dev["kc"], dev["vc"], dev["kv_len"], split_keys=split_keys,
                        scale=scale)
    torch.cuda.synchronize()
    return o.cpu().numpy()


def _oracle(q, kc, vc, lens, scale=None):
    B, H, Lmax, D = kc.shape
    o, _ = oracle.attn_fwd(q.reshape(B * H, 1, D), kc.reshape(B * H, Lmax, D),
                           vc.reshape(B * H, Lmax, D), scale=scale, causal=False,
                           kv_len=np.maximum(lens, 1), H=H)
    return o.reshape(B, H, D)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("q_bf16", [True, False])
def test_decode_small(D, q_bf16):
    B, H, Lmax = 5, 3, 700
    lens = [1, 63, 64, 513, 700]
    q, kc, vc, lens, dev = _case(B, H, Lmax, D, lens, 100 + D, q_bf16)
    say(f"decode_small D={D} q_bf16={q_bf16}")
    o = _run(dev)
    assert_close(o, _oracle(q, kc, vc, lens), "fp32", "decode O")


def test_decode_split_invariance_and_padding():
    """Any split size gives the same result; padded cache rows are never read
    (scrambling them changes nothing, bit for bit)."""
    B, H, Lmax, D = 4, 2, 2048, 128
    lens = [5, 777, 1024, 2048]
    q, kc, vc, lens, dev = _case(B, H, Lmax, D, lens, 7)
    ref = _oracle(q, kc, vc, lens)
    outs = {}
    for sk in (64, 128, 512, 2048):
        outs[sk] = _run(dev, split_keys=sk)
        assert_close(outs[sk], ref, "fp32", f"decode split={sk}")
    for b in range(B):
        dev["kc"][b, :, lens[b]:] = 1e4
        dev["vc"][b, :, lens[b]:] = -1e4
    o2 = _run(dev, split_keys=512)
    assert np.array_equal(o2, outs[512])


def test_decode_zero_length_gives_zero():
    B, H, Lmax, D = 3, 2, 256, 128
    q, kc, vc, lens, dev = _case(B, H, Lmax, D, [0, 10, 0], 9)
    o = _run(dev)
    assert np.all(o[0] == 0) and np.all(o[2] == 0)
    assert_close(o[1], _oracle(q, kc, vc, lens)[1], "fp32", "decode len=10")


def test_c4_decode_full_size():
    """C4: B=64 H=32 D=128, cache of 8192 positions, lens ~ U[512, 8192].

    The caches are drawn on the device (torch's seeded generator, bf16); the
    oracle checks every one of the 2048 (b, h) slices, one sequence (32
    slices) per oracle call, on the bf16 cache contents the kernel read."""
    from gonn_amd import hip
    B, H, Lmax, D = 64, 32, 8192, 128
    lens = np.random.default_rng(4).integers(512, 8193, B).astype(np.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(44)
    say("C4 build inputs")
    q = torch.randn((B, H, D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn((B, H, Lmax, D), generator=g, device="cuda", dtype=torch.bfloat16)
    vc = torch.randn((B, H, Lmax, D), generator=g, device="cuda", dtype=torch.bfloat16)
    kl = torch.from_numpy(lens).cuda()
    say("C4 run")
    o = hip.attn_decode(q, kc, vc, kl)
    torch.cuda.synchronize()
    o = o.cpu().numpy()
    assert np.all(np.isfinite(o))
    qn = q.float().cpu().numpy()
    worst = 0.0
    for b in range(B):
        n = int(lens[b])
        ks = kc[b, :, :n].float().cpu().numpy()
        vs = vc[b, :, :n].float().cpu().numpy()
        ro, _ = oracle.attn_fwd(qn[b][:, None, :], ks, vs, causal=False)
        worst = max(worst, assert_close(o[b], ro[:, 0], "fp32", f"C4 O b={b} len={n}"))
    say(f"C4: all {B * H} slices within the fp32 bar, worst max-abs {worst:.3e}")
