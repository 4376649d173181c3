"""GPU test of gonn_hip_attn_decode_noalloc, the decode entry point that
allocates nothing (its split partials live in a library-owned device array).

It runs the same kernels as gonn_hip_attn_decode, so on the same inputs its
output must be bit-identical to that entry point's; both are also held to the
decode bar against the oracle. Two calls in a row, the second on a smaller
input, check that the scratch array's leftover contents from the first call do
not leak into the second.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_round, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _inputs(B, H, Lmax, D, lens, seed):
    q = bf16_round(randn((B, H, D), seed))
    kc = bf16_round(randn((B, H, Lmax, D), seed + 1))
    vc = bf16_round(randn((B, H, Lmax, D), seed + 2))
    lens = np.asarray(lens, dtype=np.int32)
    dev = dict(q=torch.from_numpy(q).cuda().to(torch.bfloat16),
               kc=torch.from_numpy(kc).cuda().to(torch.bfloat16),
               vc=torch.from_numpy(vc).cuda().to(torch.bfloat16),
               kv_len=torch.from_numpy(lens).cuda())
    return q, kc, vc, lens, dev


def _noalloc(dev, split_keys=0):
    from gonn_amd import _lib, hip
    B, H, Lmax, D = dev["kc"].shape
    out = torch.full((B, H, D), float("nan"), dtype=torch.float32, device="cuda")
    a = _lib.DecodeArgs(hip.buf(dev["q"]), hip.buf(dev["kc"]), hip.buf(dev["vc"]),
                        hip.buf(dev["kv_len"]), hip.buf(out), B, H, Lmax, D,
                        1.0 / math.sqrt(D), int(split_keys))
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().gonn_hip_attn_decode_noalloc(ctypes.byref(a), st), "decode_noalloc")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _with_ws(dev, split_keys=0):
    from gonn_amd import hip
    o = hip.attn_decode(dev["q"], dev["kc"], dev["vc"], dev["kv_len"], split_keys=split_keys)
    torch.cuda.synchronize()
    return o.cpu().numpy()


def _oracle(q, kc, vc, lens):
    B, H, Lmax, D = kc.shape
    o, _ = oracle.attn_fwd(q.reshape(B * H, 1, D), kc.reshape(B * H, Lmax, D),
                           vc.reshape(B * H, Lmax, D), causal=False,
                           kv_len=np.maximum(lens, 1), H=H)
    return o.reshape(B, H, D)


@pytest.mark.parametrize("D", [64, 128])
def test_noalloc_decode_matches_workspace_entry(D):
    # First call: larger batch and cache; second: smaller, so the scratch
    # array still holds the first call's partials where the second reads none.
    cases = [(6, 4, 1500, [1, 700, 1500, 512, 64, 1024], 11),
             (2, 3, 600, [600, 65], 12)]
    for B, H, Lmax, lens, seed in cases:
        say(f"noalloc decode D={D} B={B} H={H} Lmax={Lmax} lens={lens}")
        q, kc, vc, lens, dev = _inputs(B, H, Lmax, D, lens, seed + D)
        got = _noalloc(dev)
        ref = _with_ws(dev)
        assert np.array_equal(got, ref), f"max diff {np.abs(got - ref).max()}"
        assert_close(got, _oracle(q, kc, vc, lens), "fp32", "noalloc decode O")
        # zero-length sequences give o = 0 on both entry points
        lens0 = lens.copy()
        lens0[0] = 0
        dev["kv_len"] = torch.from_numpy(lens0).cuda()
        got0 = _noalloc(dev, split_keys=128)
        ref0 = _with_ws(dev, split_keys=128)
        assert np.array_equal(got0, ref0)
        assert np.all(got0[0] == 0.0)


def test_noalloc_decode_full_size_c4_slice():
    """A C4-shaped call (B=64, H=32, Lmax=8192, D=128) fits the scratch array;
    the output equals the workspace entry's bit for bit."""
    from gonn_amd import _lib
    B, H, Lmax, D = 64, 32, 8192, 128
    rng = np.random.default_rng(4)
    lens = rng.integers(512, 8193, size=B).astype(np.int32)
    gen = torch.Generator(device="cuda").manual_seed(4)
    dev = dict(q=torch.randn((B, H, D), device="cuda", generator=gen).to(torch.bfloat16),
               kc=torch.randn((B, H, Lmax, D), device="cuda", generator=gen).to(torch.bfloat16),
               vc=torch.randn((B, H, Lmax, D), device="cuda", generator=gen).to(torch.bfloat16),
               kv_len=torch.from_numpy(lens).cuda())
    a = _lib.DecodeArgs()
    a.B, a.H, a.Lmax, a.D = B, H, Lmax, D
    need = _lib.load().gonn_hip_attn_workspace_bytes(_lib.GONN_OP_DECODE, ctypes.byref(a))
    assert need <= _lib.NOALLOC_SCRATCH_BYTES
    say("noalloc decode C4 shape")
    got = _noalloc(dev)
    ref = _with_ws(dev)
    assert np.array_equal(got, ref)
    del dev
    torch.cuda.empty_cache()


def test_noalloc_decode_allocates_nothing(monkeypatch):
    """The entry point's contract: no allocation. (1) With GONN_HIP_FAIL_ALLOC=1
    every allocation helper of the library fails (GONN_E_INJECTED), yet the
    call still succeeds with the same output. (2) It records into a graph
    under global stream capture, where a device allocation, a memset or a
    synchronisation would fail the capture; each replay, with eager work of
    the workspace entry between replays, reproduces the eager output bit for
    bit."""
    from gonn_amd import _lib, hip
    B, H, Lmax, D = 4, 3, 900, 128
    q, kc, vc, lens, dev = _inputs(B, H, Lmax, D, [5, 300, 900, 64], 31)
    ref = _noalloc(dev)  # warm-up: the per-device scratch lookup happens here
    assert_close(ref, _oracle(q, kc, vc, lens), "fp32", "noalloc decode O")
    monkeypatch.setenv("GONN_HIP_FAIL_ALLOC", "1")
    say("noalloc decode with allocation failures injected")
    assert np.array_equal(_noalloc(dev), ref)
    monkeypatch.delenv("GONN_HIP_FAIL_ALLOC")

    out = torch.full((B, H, D), float("nan"), dtype=torch.float32, device="cuda")
    a = _lib.DecodeArgs(hip.buf(dev["q"]), hip.buf(dev["kc"]), hip.buf(dev["vc"]),
                        hip.buf(dev["kv_len"]), hip.buf(out), B, H, Lmax, D,
                        1.0 / math.sqrt(D), 0)
    lib = _lib.load()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    say("noalloc decode under graph capture")
    with torch.cuda.graph(graph, stream=side, capture_error_mode="global"):
        rc = lib.gonn_hip_attn_decode_noalloc(
            ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _lib.strerror(rc)
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), ref), f"replay {i}"
        assert np.array_equal(_with_ws(dev), ref)
