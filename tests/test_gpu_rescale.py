"""GPU parity on planted-peak inputs: the forward kernels' lazy-rescale paths.

The bf16 forward keeps a running offset mc per query (the first tile's row
max) and only moves it when a later 64-key tile's row sum, taken relative to
mc, exceeds 2^14 or is not finite (attn_fwd.hip: the unmasked pipelined
kernel's `!(ts <= kSumBound)` branch, the masked pipelined kernel's branch,
and the two-stage kernel's `grow` test at kLazyLog2). With N(0,1) inputs a
later tile's maximum sits only a few log2 units above tile 0's, so none of
these branches runs; real attention takes them whenever a late key matches a
query much better than every earlier key.

Inputs: Q = N(0,1) + 0.5, so sum_d Q_d is about D/2 for every query; the K
rows of chosen tiles get a constant added (a "plant"), which raises every
score against those keys by about scale * D/2 * shift. The shifts grow from
plant to plant, so each planted tile moves the row maximum by 8 to 30 nat
(12 to 43 log2 units) over the previous one: each one takes the branch. One
case adds a tile about 100 nat above the rest, where exp2 of the score
relative to mc overflows fp32 (the row sum is +inf, the branch's "not
finite" arm). Plants sit on tile 1 (handled by the first pipeline step),
middle tiles, and the last tile of a block (the next-to-last pipeline step).

Each case runs both MFMA modes, forward (O, LSE) against the fp64 oracle on
every row, and the backward against the oracle's autograd chain (GoNN's
nn/attention.go:107-148 and tensor/autograd.go:52-151 restated), at the
stated bars. An all-zero additive mask routes the same inputs through the
masked kernels (their own rescale branch) with identical expected results.

Which inputs the oracle sees: fp32 mode, the inputs themselves. bf16 mode,
the operands the kernels read: Q * scale * log2(e) rounded to bf16 (divided
back by that factor), K, V and dO rounded to bf16. On planted inputs a row's
weight sits on a handful of keys of one tile, and the rounding of the inputs
alone moves O by up to 2.6e-2 (an fp64 evaluation on the rounded operands,
with P rounded to bf16, reproduces the kernel's output there to 1e-7; the
oracle on the rounded operands is within 2.8e-3 of it), past the bf16 bar,
which is stated for the N(0,1) configs. Against the rounded operands the
kernel's own error (bf16 P and dS, fp32 sums) is what the bar measures; a
mistake in a rescale branch (a wrong offset, a missed shift of the tile in
flight, O or l not rescaled) weighs a tile by a factor 2^8 or more wrong and
fails it by orders of magnitude.
"""
import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_round, randn, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


# Mean of Q: the common direction the planted K offsets align with.
Q_MEAN = 0.5


def _planted(BH, Sq, Sk, D, seed, plants):
    """Q = N(0,1) + Q_MEAN; K with a constant added to the rows of each
    planted tile (64 keys from tile*64); V, dO = N(0,1). `plants` holds
    (tile, nat): the planted tile's scores rise by about `nat` over the
    unplanted ones."""
    q = randn((BH, Sq, D), seed) + np.float32(Q_MEAN)
    k = randn((BH, Sk, D), seed + 1)
    v = randn((BH, Sk, D), seed + 2)
    g = randn((BH, Sq, D), seed + 3)
    # sum_d q_d ~ Q_MEAN D, so a shift c on every K element adds c Q_MEAN sqrt(D).
    per_unit = Q_MEAN * D / np.sqrt(D)
    for tile, nat in plants:
        lo, hi = tile * 64, min(Sk, tile * 64 + 64)
        if lo < Sk:
            k[:, lo:hi] += np.float32(nat / per_unit)
    return q, k, v, g


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _operands(mode, D, q, k, v, g=None):
    """The values the kernels of `mode` compute with (see the module text)."""
    if mode == "fp32":
        return q, k, v, g
    c2 = np.float32(1.0 / np.sqrt(D) * np.log2(np.e))
    qr = bf16_round(q * c2).astype(np.float64) / np.float64(c2)
    return (qr, bf16_round(k), bf16_round(v), None if g is None else bf16_round(g))


CASES = {
    # (Sq, Sk, plants): plants rise 12 nat, then 24, ... over the base scores
    "S200": (200, 200, [(1, 12.0), (3, 24.0)]),
    "S1024": (1024, 1024, [(1, 10.0), (3, 20.0), (8, 31.0), (15, 42.0)]),
    "S4096": (4096, 4096, [(1, 10.0), (3, 20.0), (10, 31.0), (30, 42.0), (63, 53.0)]),
    "overflow": (640, 640, [(2, 12.0), (6, 100.0)]),
    "cross": (300, 1000, [(1, 12.0), (9, 25.0), (15, 38.0)]),
}


def _check_fwd(name, D, causal, mode, masked):
    from gonn_amd import hip
    Sq, Sk, plants = CASES[name]
    BH = 2
    q, k, v, _ = _planted(BH, Sq, Sk, D, 9100 + D + Sq, plants)
    mask = torch.zeros((Sq, Sk), device="cuda") if masked else None
    say(f"[rescale fwd] {name} D={D} causal={causal} mode={mode} masked={masked}")
    o, l = hip.attn_fwd(_dev(q), _dev(k), _dev(v), causal=causal, mode=mode, attn_mask=mask)
    torch.cuda.synchronize()
    qo, ko, vo, _ = _operands(mode, D, q, k, v)
    ro, rl = oracle.attn_fwd(qo, ko, vo, causal=causal)
    # the plants do move the row maxima far from tile 0's (else the case
    # would not reach the branch)
    assert float(np.max(rl)) - float(np.min(rl[:, :64])) > 20.0
    assert_close(o.cpu().numpy(), ro, mode, f"{name} O")
    assert_close(l.cpu().numpy(), rl, mode, f"{name} LSE")


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("name", ["S200", "S4096", "overflow", "cross"])
def test_rescale_fwd(name, causal, D, mode):
    _check_fwd(name, D, causal, mode, masked=False)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("name", ["S200", "S1024", "overflow"])
def test_rescale_fwd_masked_kernels(name, causal, D):
    """An all-zero (Sq, Sk) additive mask: the same results through the
    masked bf16 kernels, whose offsets stay out of the accumulators."""
    _check_fwd(name, D, causal, "bf16", masked=True)


@pytest.mark.parametrize("mode", ["bf16", "fp32"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("name", ["S200", "S1024", "overflow"])
def test_rescale_bwd(name, causal, D, mode):
    """Backward from the forward's own O and LSE on the planted inputs.

    The backward kernels have no rescale branch (they read the forward's
    LSE); this runs them on the scores the branch produces.

    fp32 mode: the 1e-4 bar, except the overflow case, which stays at the
    fp32 forward's check (test_rescale_fwd): its scores reach ~160 nat, where
    exp(s - L) formed from fp32 s and L carries a relative error of about
    |s| * 2^-23 ~ 2e-5, which alone moves dV by ~1e-4 (seen: 1.07e-4).

    bf16 mode: the planted offsets lift the gradients to |dQ| ~ 2-3, |dK| and
    |dV| ~ 3-11 (N(0,1) configs: ~1), and two bf16 effects scale with them:
    the planted K offset c multiplies the row sums of dS (zero in exact
    arithmetic, ~1e-2 once the forward's bf16 P and the backward's P and dS
    roundings differ) into dQ = scale sum_j dS_ij K_j, and P, dS rounded to
    bf16 carry 2^-9 of each term. The bar adds 2% of the tensor's largest
    magnitude to the stated one: |got - ref| <= 2e-2 + 1e-2 |ref| +
    2e-2 max|ref| (seen: up to 1.6% of max|dQ|). A wrong or missing term
    (a tile dropped or doubled, a wrong LSE) moves a gradient by a sizeable
    fraction of max|ref| and still fails."""
    if mode == "fp32" and name == "overflow":
        return
    from gonn_amd import hip
    Sq, Sk, plants = CASES[name]
    BH = 2
    q, k, v, g = _planted(BH, Sq, Sk, D, 9200 + D + Sq, plants)
    say(f"[rescale bwd] {name} D={D} causal={causal} mode={mode}")
    dq_, dk_, dv_, dg_ = _dev(q), _dev(k), _dev(v), _dev(g)
    o, l = hip.attn_fwd(dq_, dk_, dv_, causal=causal, mode=mode)
    dq, dk, dv = hip.attn_bwd(dq_, dk_, dv_, o, l, dg_, causal=causal, mode=mode)
    torch.cuda.synchronize()
    rq, rk, rv = oracle.attn_bwd_autograd(*_operands(mode, D, q, k, v, g), causal=causal)
    for got, ref, what in ((dq, rq, "dQ"), (dk, rk, "dK"), (dv, rv, "dV")):
        got = got.cpu().numpy().astype(np.float64)
        if mode == "fp32":
            assert_close(got, ref, mode, f"{name} {what}")
            continue
        err = np.abs(got - ref)
        bound = 2e-2 + 1e-2 * np.abs(ref) + 2e-2 * np.abs(ref).max()
        say(f"[{name} {what}] bf16 max_abs={err.max():.3e} max|ref|={np.abs(ref).max():.3f} "
            f"worst err/bound={(err / bound).max():.3f}")
        assert np.all(np.isfinite(got)) and np.all(err <= bound), what


def test_planted_inputs_reach_the_branch():
    """CPU check of the construction (no GPU call): on the oracle's scores, in
    log2 units relative to tile 0's row max, some later 64-key tile's row
    sum exceeds 2^14 for most rows that see a plant, and the overflow case
    holds a tile whose exp2 relative to tile 0's max is past fp32 range."""
    for name in ("S200", "S4096", "overflow"):
        Sq, Sk, plants = CASES[name]
        D = 128
        q, k, _, _ = _planted(1, Sq, Sk, D, 9100 + D + Sq, plants)
        s = (q[0].astype(np.float64) @ k[0].astype(np.float64).T) / np.sqrt(D) * np.log2(np.e)
        first = plants[0][0] * 64
        rows = np.arange(first + 64, Sq)
        mc = s[rows, :64].max(axis=1, keepdims=True)
        big = np.zeros(len(rows), bool)
        for tile, _ in plants:
            lo, hi = tile * 64, min(Sk, tile * 64 + 64)
            if lo >= Sk:
                continue
            ts = np.exp2(np.minimum(s[rows, lo:hi] - mc, 1000)).sum(axis=1)
            big |= ts > 2.0 ** 14
        assert big.mean() > 0.9, (name, big.mean())
        if name == "overflow":
            assert (s[rows, 6 * 64:7 * 64] - mc).max() > 128
