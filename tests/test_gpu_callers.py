"""GPU parity of the attention core's callers, through the differentiable
fused node (MultiHeadAttention.forward + last_node, nn/attention.go:107-148
with fusedAttnDiff at :129-133) in the three call patterns of GoNN's
transformer layers:

  encoder            Attn.Forward(x, x, x, false)           nn/transformer.go:124-136
  decoder self       SelfAttn.Forward(t, t, t, true)        nn/transformer.go:232
  decoder cross      CrossAttn.Forward(x, mem, mem, false)  nn/transformer.go:234 (Tq != Tk)

Each runs at D = 64 and 128 in both MFMA modes. The layer output is checked
against the oracle's MultiHeadAttention (oracle.mha_fwd, fp64), and the node's
gradients of the projected heads against the oracle's autograd chain
(oracle.attn_bwd_autograd, rectangular for cross-attention), at the mode's
bar (tests/_util.py TOL). The inputs are N(0,1) and the weights
N(0,1)/sqrt(E), so the projected heads the core sees are O(1) as in C2-C5;
one C1-scaled case (inputs and weights N(0,1)/sqrt(E)) runs as well.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import assert_close, randn, say

pytestmark = pytest.mark.gpu


def _layer(E, H, seed, x_scale=1.0):
    from gonn_amd import nn
    rng = np.random.default_rng(seed)
    ws = 1.0 / math.sqrt(E)
    p = {}
    for n in ("q", "k", "v", "o"):
        p["W" + n] = rng.standard_normal((E, E)) * ws
        p["b" + n] = rng.standard_normal(E) * 0.1 * x_scale
    mha = nn.MultiHeadAttention(E, H, p["Wq"], p["bq"], p["Wk"], p["bk"], p["Wv"], p["bv"],
                                p["Wo"], p["bo"])
    return mha, p


PATTERNS = {
    # name: (Tq, Tk, causal, kv from memory)
    "encoder": (80, 80, False, False),
    "decoder_self": (56, 56, True, False),
    "decoder_cross": (56, 100, False, True),
}


def _run(pattern, D, mode, x_scale=1.0, seed=0):
    from gonn_amd import hip
    Tq, Tk, causal, cross = PATTERNS[pattern]
    B, H = 2, 2
    E = H * D
    mha, p = _layer(E, H, 7000 + D + seed, x_scale)
    rng = np.random.default_rng(8000 + D + seed)
    x = rng.standard_normal((B, Tq, E)) * x_scale
    mem = rng.standard_normal((B, Tk, E)) * x_scale if cross else x
    g = randn((B * H, Tq, D), 9000 + D + seed).astype(np.float64)
    prev = hip.AttnMode()
    hip.SetAttnMode(mode)
    try:
        say(f"[callers] {pattern} D={D} mode={mode} Tq={Tq} Tk={Tk} causal={causal}")
        out = mha.forward(x, mem, mem, causal)
        node = mha.last_node
        dq, dk, dv = node(g.ravel())
    finally:
        hip.SetAttnMode(prev)
    ref = oracle.mha_fwd(x, mem, mem, p, H, causal=causal)
    assert_close(out, ref, mode, f"{pattern} D={D} out")
    qp = oracle.split_heads(oracle.linear(x, p["Wq"], p["bq"]), H)
    kp = oracle.split_heads(oracle.linear(mem, p["Wk"], p["bk"]), H)
    vp = oracle.split_heads(oracle.linear(mem, p["Wv"], p["bv"]), H)
    rq, rk, rv = oracle.attn_bwd_autograd(qp, kp, vp, g, scale=1.0 / math.sqrt(D), causal=causal)
    assert_close(dq.reshape(B * H, Tq, D), rq, mode, f"{pattern} D={D} dQ")
    assert_close(dk.reshape(B * H, Tk, D), rk, mode, f"{pattern} D={D} dK")
    assert_close(dv.reshape(B * H, Tk, D), rv, mode, f"{pattern} D={D} dV")


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("pattern", list(PATTERNS))
def test_transformer_call_patterns(pattern, D, mode):
    _run(pattern, D, mode)


@pytest.mark.parametrize("pattern", list(PATTERNS))
def test_c1_scaled_call_patterns(pattern):
    """BASELINE C1's scaling: inputs and weights N(0,1)/sqrt(d_model)."""
    _run(pattern, 64, "fp32", x_scale=1.0 / math.sqrt(128), seed=1)
