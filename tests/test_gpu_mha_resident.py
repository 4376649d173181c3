"""GPU parity of the device-resident multi-head attention (gonn_hip_mha_*:
nn.MultiHeadAttention's forward, nn/attention.go:107-148, with weights and
intermediates in HBM) against the oracle's fp64 MHA and against the
host-projection path of the same layer.

Bars: the oracle at the arithmetic mode's bar (fp32-MFMA max-abs 1e-4;
bf16-MFMA 2e-2 + 1e-2|ref|); the host-projection path with the projections on
the HIP backend (same rocBLAS GEMMs, same fused core) at 1e-12."""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _layer(E, H, kdim, vdim, seed, bias=True):
    from gonn_amd import nn
    s = 1.0 / math.sqrt(E)
    p = {"Wq": randn((E, E), seed).astype(np.float64) * s,
         "Wk": randn((E, kdim), seed + 1).astype(np.float64) / math.sqrt(kdim),
         "Wv": randn((E, vdim), seed + 2).astype(np.float64) / math.sqrt(vdim),
         "Wo": randn((E, E), seed + 3).astype(np.float64) * s}
    for i, n in enumerate("qkvo"):
        p["b" + n] = randn((E,), seed + 10 + i).astype(np.float64) * 0.1 if bias else np.zeros(E)
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"] if bias else None, p["Wk"],
                                p["bk"] if bias else None, p["Wv"], p["bv"] if bias else None,
                                p["Wo"], p["bo"] if bias else None)
    return mha, p


@pytest.fixture
def mode_guard():
    from gonn_amd import hip
    prev = hip.AttnMode()
    yield hip
    hip.SetAttnMode(prev)


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("cfg", [
    ("C1", 2, 128, 128, 256, 4, True),        # self-attention, causal
    ("D128 ragged", 2, 77, 77, 512, 4, True),
    ("D32 padded", 3, 50, 50, 128, 4, False),
], ids=lambda c: c[0] if isinstance(c, tuple) else c)
def test_resident_self_attention_matches_oracle(mode_guard, mode, cfg):
    from gonn_amd import backend
    hip = mode_guard
    name, B, Tq, Tk, E, H, causal = cfg
    say(f"[mha resident] {name} mode={mode}")
    hip.SetAttnMode(mode)
    mha, p = _layer(E, H, E, E, 1000 + E)
    x = randn((B, Tq, E), 1100 + Tq).astype(np.float64)
    if name == "C1":
        x /= math.sqrt(E)  # inputs N(0,1) / sqrt(d_model)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=causal)
    with mha.to_device() as dev:
        got = dev.forward(x, x, x, causal)
    assert_close(got, ref, mode, f"resident MHA {name}")
    prev = backend.Use(backend.HIPBackend())
    try:
        host = mha.forward_fused(x, x, x, causal)
    finally:
        backend.Use(prev)
    assert np.max(np.abs(got - host)) <= 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_resident_cross_attention_and_key_padding(mode_guard, causal):
    hip = mode_guard
    hip.SetAttnMode("fp32")
    B, Tq, Tk, E, H, kdim, vdim = 3, 40, 90, 256, 4, 96, 160
    say(f"[mha resident] cross causal={causal}")
    mha, p = _layer(E, H, kdim, vdim, 1200)
    q = randn((B, Tq, E), 1201).astype(np.float64)
    k = randn((B, Tk, kdim), 1202).astype(np.float64)
    v = randn((B, Tk, vdim), 1203).astype(np.float64)
    lens = [90, 33, 61]
    pad = np.zeros((B, Tk))
    for b, n in enumerate(lens):
        pad[b, n:] = 1.0
    with mha.to_device() as dev:
        got = dev.forward(q, k, v, causal)
        gotm = dev.forward_masked(q, k, v, causal, key_padding_mask=pad)
        with pytest.raises(ValueError):
            holes = pad.copy()
            holes[1, 5] = 1.0
            dev.forward_masked(q, k, v, causal, key_padding_mask=holes)
    assert_close(got, oracle.mha_fwd(q, k, v, p, H, causal=causal), "fp32", "resident cross")
    assert_close(gotm, oracle.mha_fwd(q, k, v, p, H, causal=causal, key_pad=pad), "fp32",
                 "resident cross + key padding")
    assert np.max(np.abs(gotm - mha.forward_masked(q, k, v, causal, key_padding_mask=pad))) <= 1e-9


def test_resident_without_bias(mode_guard):
    hip = mode_guard
    hip.SetAttnMode("fp32")
    mha, p = _layer(128, 2, 128, 128, 1300, bias=False)
    x = randn((2, 33, 128), 1301).astype(np.float64)
    with mha.to_device() as dev:
        got = dev.forward(x, x, x, True)
    assert_close(got, oracle.mha_fwd(x, x, x, p, 2, causal=True), "fp32", "resident, no bias")


def test_resident_device_buffers_reuse_workspace(mode_guard):
    """forward_dev on torch tensors with one caller workspace, two calls in a
    row (the second smaller), equals the host-data entry bit for bit."""
    hip = mode_guard
    hip.SetAttnMode("bf16")
    E, H = 256, 2
    mha, p = _layer(E, H, E, E, 1400)
    with mha.to_device() as dev:
        need = dev.dev.workspace_bytes(2, 256, 256)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        for (B, T) in ((2, 256), (1, 100)):
            x = randn((B, T, E), 1401 + T).astype(np.float64)
            xd = torch.from_numpy(x).cuda()
            assert dev.dev.workspace_bytes(B, T, T) <= need
            out = dev.dev.forward_dev(xd, xd, xd, causal=True, ws=ws)
            torch.cuda.synchronize()
            host = dev.forward(x, x, x, True)
            assert np.array_equal(out.cpu().numpy(), host), (B, T)
            assert_close(host, oracle.mha_fwd(x, x, x, p, H, causal=True), "bf16", f"resident dev {B}x{T}")
        kl = torch.tensor([50], dtype=torch.int32, device="cuda")
        out = dev.dev.forward_dev(xd, xd, xd, causal=False, kv_len=kl, ws=ws)
        torch.cuda.synchronize()
        pad = np.zeros((1, 100))
        pad[0, 50:] = 1
        assert np.array_equal(out.cpu().numpy(), dev.forward_masked(x, x, x, False, key_padding_mask=pad))
        with pytest.raises(Exception):
            dev.dev.forward_dev(xd, xd, xd, ws=ws[:16])


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_resident_forward_dev_graph_replay(mode_guard, mode):
    """The device-resident forward allocates nothing and only launches
    kernels on the caller's stream, so a caller can capture it in a HIP
    graph (here torch's CUDAGraph) and replay it. C1's shape (both
    projections on the skinny fp64 GEMM kernel): three replays, each after
    new inputs are copied into the captured buffer and with eager calls and
    synchronisations in between, each bit-identical to an eager call on the
    same inputs; the eager result is checked against the oracle."""
    hip = mode_guard
    hip.SetAttnMode(mode)
    B, S, E, H = 2, 128, 256, 4
    mha, p = _layer(E, H, E, E, 1500)
    with mha.to_device() as dev:
        ws = torch.empty(dev.dev.workspace_bytes(B, S, S), dtype=torch.uint8, device="cuda")
        ws2 = torch.empty_like(ws)
        xs = [randn((B, S, E), 1501 + i).astype(np.float64) / math.sqrt(E) for i in range(3)]
        xd = torch.from_numpy(xs[0]).cuda()
        out = torch.empty_like(xd)
        dev.dev.forward_dev(xd, xd, xd, out=out, causal=True, ws=ws)  # eager first call
        torch.cuda.synchronize()
        say(f"[mha resident] graph capture mode={mode}")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            dev.dev.forward_dev(xd, xd, xd, out=out, causal=True, ws=ws)
        for i, x in enumerate(xs):
            xe = torch.from_numpy(x).cuda()
            xd.copy_(xe)
            g.replay()
            torch.cuda.synchronize()
            got = out.clone()
            ref = dev.dev.forward_dev(xe, xe, xe, causal=True, ws=ws2)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"replay {i}"
            assert_close(ref.cpu().numpy(), oracle.mha_fwd(x, x, x, p, H, causal=True), mode,
                         f"graph replay {i}")


def test_resident_layer_in_the_f64_entries_mode(mode_guard):
    """With the f64 entries' fp64 mode set, the resident layer still runs
    (its core on fp32-MFMA over its fp32 intermediates)."""
    hip = mode_guard
    hip.SetAttnMode("f64")
    E, H, B, T = 256, 4, 2, 128
    mha, p = _layer(E, H, E, E, 1256)
    x = randn((B, T, E), 1257).astype(np.float64) / math.sqrt(E)
    ref = oracle.mha_fwd(x, x, x, p, H, causal=True)
    with mha.to_device() as dev:
        got = dev.forward(x, x, x, True)
    assert_close(got, ref, "fp32", "resident MHA in f64 mode")
    # the host-data fused path of the same layer runs the fp64 kernels
    assert np.max(np.abs(mha.forward_fused(x, x, x, True) - ref)) <= 1e-9
