"""gonn_amd.nn -- the nn-level attention seam on the HIP backend.

Mirrors GoNN's build-tagged seam nn/flashattn_cuda.go (what a Go maintainer
adds as nn/flashattn_hip.go) and the fused branch of
MultiHeadAttention.Forward / ForwardFused (nn/attention.go:107-180):

    fused_attn_available()                         nn/flashattn_cuda.go:13
    fused_attn_supports(D, Tq, Tk)                 gate of nn/attention.go:129
    fused_attn_f64(Q, K, V, BH, S, D, scale, c)    nn/flashattn_cuda.go:17-21
    fused_attn_diff(qp, kp, vp, BH, S, D, scale, c)nn/flashattn_cuda.go:26-38
    MultiHeadAttention.forward / forward_fused     nn/attention.go:107-148, :159-180

Tensors are host float64 arrays as in GoNN (tensor/tensor.go:22-23); the
projections and the output projection run on the host in fp64 exactly like
the reference's fused path (nn/attention.go:115-117, :132), and the core runs
in the HIP kernels. There is no CPU fallback for the core: when the HIP
library or device is missing, these functions raise, like the reference's
non-cuda stubs panic (nn/flashattn_nocuda.go:12-20).
"""
from __future__ import annotations

import math

import numpy as np

from . import backend, hip


def fused_attn_available() -> bool:
    return hip.Available()


def fused_attn_supports(D: int, Tq: int, Tk: int) -> bool:
    return hip.Supports(D, Tq, Tk)


def fused_attn_f64(Q, K, V, BH: int, S: int, D: int, scale: float, causal: bool) -> np.ndarray:
    """Inference forward of the core on flat (BH,S,D) float64 data."""
    O = np.zeros(BH * S * D)
    hip.FlashAttnF64(Q, K, V, O, BH, S, D, scale, causal)
    return O


class FusedAttnNode:
    """The autograd node fusedAttnDiff attaches (MakeNode "FlashAttn",
    nn/flashattn_cuda.go:29-37): holds what the backward needs and runs the
    device backward when called with the upstream gradient."""

    def __init__(self, Q, K, V, O, L, BH, S, D, scale, causal, kv_len=None, H=1, attn_mask=None,
                 Sk=None):
        self.saved = (Q, K, V, O, L)
        self.shape = (BH, S, D)
        self.Sk = S if Sk is None else int(Sk)
        self.scale = scale
        self.causal = causal
        self.kv_len, self.H, self.attn_mask = kv_len, H, attn_mask

    def plain(self) -> bool:
        """The reference seam's own case: square, no padding, no mask."""
        return self.kv_len is None and self.attn_mask is None and self.Sk == self.shape[1]

    def __call__(self, grad):
        Q, K, V, O, L = self.saved
        BH, S, D = self.shape
        if self.plain():
            return hip.FlashAttnF64Bwd(Q, K, V, O, L, grad, BH, S, D, self.scale, self.causal)
        return hip.FlashAttnF64BwdEx(Q, K, V, O, L, grad, BH // self.H, self.H, S, D,
                                     self.scale, self.causal, kv_len=self.kv_len,
                                     attn_mask=self.attn_mask, Sk=self.Sk)


def fused_attn_diff(qp, kp, vp, BH: int, S: int, D: int, scale: float, causal: bool,
                    kv_len=None, H: int = 1, attn_mask=None, Sk=None):
    """Differentiable core: returns (O, node) where node(dO) -> (dQ, dK, dV).
    kv_len (new): optional per-sequence key counts (BH / H entries), the key
    padding of ForwardMasked; attn_mask (new): its additive mask; Sk (new):
    the key rows of kp and vp when they differ from S (cross-attention, top-
    left causal mask); all in the forward and the backward."""
    Sk = S if Sk is None else int(Sk)
    node = FusedAttnNode(np.ascontiguousarray(qp, dtype=np.float64).ravel(),
                         np.ascontiguousarray(kp, dtype=np.float64).ravel(),
                         np.ascontiguousarray(vp, dtype=np.float64).ravel(), None, None, BH, S, D,
                         scale, causal, kv_len, H, attn_mask, Sk)
    Q, K, V = node.saved[:3]
    if node.plain():
        O, L = hip.FlashAttnF64Fwd(Q, K, V, BH, S, D, scale, causal)
    else:
        O, L = hip.FlashAttnF64Ex(Q, K, V, BH // H, H, S, Sk, D, scale, causal,
                                  kv_len=kv_len, lse=True, attn_mask=attn_mask)
    node.saved = (Q, K, V, O, L)
    return O, node


class Linear:
    """y = x @ W^T + b (nn/linear.go:40-59); W is (out, in)."""

    def __init__(self, W, b=None):
        self.W = np.asarray(W, dtype=np.float64)
        self.b = None if b is None else np.asarray(b, dtype=np.float64)

    def forward(self, x):
        # x2 @ W^T through the current backend (tensor.MatMul -> dispatchGemm,
        # tensor/dispatch.go:111-113): W is stored (out, in), so op(B) = W^T.
        x = np.asarray(x, dtype=np.float64)
        out, inp = self.W.shape
        x2 = x.reshape(-1, inp)
        y = backend.Current().Gemm(x2, self.W, 1, x2.shape[0], inp, out, False, True)
        y = y.reshape(x2.shape[0], out)
        if self.b is not None:
            y = y + self.b
        return y.reshape(*x.shape[:-1], out)


# A row of the core whose best in-window additive mask value is at or below
# NO_KEY_LEVEL has no unblocked key. GoNN adds its masks as -1e30 constants
# (nn/attention.go:185-196, :261-272) in fp64, where they absorb the scores,
# so such a row's softmax depends on the mask sums alone: a uniform average
# over the keys whose summed mask is the row's maximum. Future keys count too,
# with their causal -1e30. The fused core reproduces it when the row's maximum
# is at or below UNIFORM_LEVEL: the scores vanish next to it in fp32 as in
# fp64, so the row is passed unshifted. A blocked row whose maximum lies
# between the two levels (fp64 keeps part of the score there, fp32 does not)
# is refused, and so is a row whose every key is -inf (NaN in the reference).
NO_KEY_LEVEL = -1e15
UNIFORM_LEVEL = -1e25
_NO_KEY_MSG = ("nn: a query row has no unblocked key (every key it may attend is padded or "
               "masked); the fused core does not define such rows")
_BLOCKED_MSG = ("nn: a query row has no unblocked key and its best mask value lies between "
                "-1e25 and -1e15 (or is -inf); the fused core does not define such rows")


def _kv_len_from_mask(key_padding_mask, B: int, Tk: int):
    """kv_len[b] of a (B, Tk) key-padding mask (nonzero = ignore the key,
    keyPaddingMaskAdd, nn/attention.go:261-272) whose padded keys are a
    suffix of each row, leaving at least one key; None for no mask. Any
    other mask raises ValueError."""
    kv_len, kp_add = _key_padding(key_padding_mask, B, Tk)
    if kp_add is not None:
        if (kp_add != 0).all(axis=1).any():
            raise ValueError(_NO_KEY_MSG)
        raise ValueError("nn: this path takes key padding masks whose padded keys are a "
                         "suffix of the row")
    return kv_len


def _key_padding(key_padding_mask, B: int, Tk: int):
    """(kv_len, None) for a suffix-form padding mask whose rows keep a key,
    (None, additive (B, Tk) 0 / -1e30 mask) for any other, (None, None) for
    none."""
    if key_padding_mask is None:
        return None, None
    m = np.asarray(key_padding_mask)
    if m.shape != (B, Tk):  # keyPaddingMaskAdd's shape check, nn/attention.go:262-264
        raise ValueError(f"MultiHeadAttention: key padding mask shape {m.shape}, "
                         f"want (B, Tk) = ({B}, {Tk})")
    pad = m != 0
    n = np.where(pad.any(axis=1), pad.argmax(axis=1), Tk)
    if all(pad[b, n[b]:].all() for b in range(B)) and n.all():
        return n.astype(np.int32), None
    return None, np.where(pad, -1e30, 0.0)


def _core_masks(key_padding_mask, attn_mask, B: int, H: int, Tq: int, Tk: int, causal: bool):
    """ForwardMasked's masks (nn/attention.go:318-330) in the form the fused
    core takes them: (kv_len or None, additive mask or None, causal).

    A suffix-form padding mask becomes kv_len (the kernels skip the padded
    keys); any other is added as keyPaddingMaskAdd's 0 / -1e30 values. Each
    row of the additive mask is shifted by its maximum over the keys the row
    attends (causal window, kv_len): softmax is unchanged, and the fp32
    scores the kernels form keep full precision under a large common offset.

    When some row has no unblocked key (that maximum at or below
    NO_KEY_LEVEL), the call takes the whole-row form instead: the causal mask
    and the key padding become the reference's -1e30 terms, added in its
    order (causal, attn_mask, key padding) over every key, the call runs
    non-causal and without kv_len, each row with an unblocked key is shifted
    by its maximum, and each blocked row stays as it is (see UNIFORM_LEVEL).
    Blocked rows the core cannot reproduce raise ValueError."""
    kv_len, kp_add = _key_padding(key_padding_mask, B, Tk)
    if attn_mask is None and kp_add is None:
        return kv_len, None, causal  # a suffix-form kv_len leaves every row a key
    if attn_mask is not None:
        sb, sh = hip.mask_strides(np.shape(attn_mask), B, H, Tq, Tk)  # expandAttnMask's check
        Hu = H if sh else 1
        user = np.asarray(attn_mask, dtype=np.float64).reshape(B if sb else 1, Hu, Tq, Tk)
        user = np.broadcast_to(user, (B, Hu, Tq, Tk))
    else:
        Hu, user = 1, np.zeros((B, 1, Tq, Tk))
    full = user if kp_add is None else user + kp_add[:, None, None, :]
    win = np.ones((B, 1, Tq, Tk), dtype=bool)
    if kv_len is not None:
        win &= (np.arange(Tk)[None, :] < kv_len[:, None])[:, None, None, :]
    if causal:
        win &= (np.arange(Tk)[None, :] <= np.arange(Tq)[:, None])[None, None]
    wmax = np.where(win, full, -np.inf).max(axis=-1)
    if (wmax > NO_KEY_LEVEL).all():
        if kp_add is None and not wmax.any():
            return kv_len, attn_mask, causal
        out = np.ascontiguousarray(full - wmax[..., None])
        return kv_len, (out[:, 0] if out.shape[1] == 1 else out), causal
    # whole-row form, in the reference's order of additions
    whole = np.zeros((B, Hu, Tq, Tk))
    if causal:
        whole = whole + np.where(np.arange(Tk)[None, :] > np.arange(Tq)[:, None], -1e30, 0.0)
    whole = whole + user
    pad = kp_add
    if kv_len is not None:
        pad = np.where(np.arange(Tk)[None, :] >= kv_len[:, None], -1e30, 0.0)
    if pad is not None:
        whole = whole + pad[:, None, None, :]
    rmax = whole.max(axis=-1)
    blocked = ~(rmax > NO_KEY_LEVEL)
    if not (np.isfinite(rmax[blocked]).all() and (rmax[blocked] <= UNIFORM_LEVEL).all()):
        raise ValueError(_BLOCKED_MSG)
    out = np.ascontiguousarray(whole - np.where(blocked, 0.0, rmax)[..., None])
    return None, (out[:, 0] if Hu == 1 else out), False


class MultiHeadAttention:
    """Forward-path mirror of nn.MultiHeadAttention with the fused core.

    Weights are given explicitly (GoNN draws them from its global math/rand
    stream, nn/linear.go:20-36, which only Go can reproduce).
    """

    def __init__(self, embed_dim: int, num_heads: int, Wq, bq, Wk, bk, Wv, bv, Wo, bo):
        if embed_dim % num_heads != 0:
            raise ValueError("MultiHeadAttention: embedDim must be divisible by numHeads")
        self.EmbedDim = embed_dim
        self.NumHeads = num_heads
        self.HeadDim = embed_dim // num_heads
        self.QProj, self.KProj = Linear(Wq, bq), Linear(Wk, bk)
        self.VProj, self.OutProj = Linear(Wv, bv), Linear(Wo, bo)

    def _check(self, q, k, v):
        # checkQKVDims, nn/attention.go:83-103
        E = self.EmbedDim
        if q.ndim != 3 or q.shape[2] != E:
            raise ValueError(f"MultiHeadAttention: q shape {q.shape}, want (B, Tq, {E})")
        if k.ndim != 3 or k.shape[2] != self.KProj.W.shape[1]:
            raise ValueError(f"MultiHeadAttention: k shape {k.shape}")
        if v.ndim != 3 or v.shape[2] != self.VProj.W.shape[1]:
            raise ValueError(f"MultiHeadAttention: v shape {v.shape}")
        if k.shape[1] != v.shape[1]:
            raise ValueError("MultiHeadAttention: k and v sequence lengths differ")

    def _split(self, x):
        B, T, _ = x.shape
        H, D = self.NumHeads, self.HeadDim
        return np.ascontiguousarray(x.reshape(B, T, H, D).transpose(0, 2, 1, 3))

    def forward_fused(self, q, k, v, causal: bool):
        """ForwardFused: projections, fused core, output projection."""
        q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
        self._check(q, k, v)
        if not fused_attn_available():
            raise RuntimeError("nn: fused attention requires the HIP library and a gfx950 device")
        return self._fused(q, k, v, causal, None)

    def forward(self, q, k, v, causal: bool):
        """Forward (nn/attention.go:107-148) with the differentiable fused
        core (fusedAttnDiff, :129-133), Tq != Tk included: the encoder's
        Forward(x, x, x, false), the decoder's causal self-attention
        Forward(t, t, t, true) and its cross-attention Forward(x, memory,
        memory, false) (nn/transformer.go:124-136, :224-238). The node of the
        call is kept in last_node: last_node(g) maps the gradient g of the
        core output (B*H, Tq, D) to the gradients of the projected heads."""
        q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
        self._check(q, k, v)
        if not fused_attn_available():
            raise RuntimeError("nn: fused attention requires the HIP library and a gfx950 device")
        B, Tq, _ = q.shape
        Tk = k.shape[1]
        H, D = self.NumHeads, self.HeadDim
        qp = self._split(self.QProj.forward(q))
        kp = self._split(self.KProj.forward(k))
        vp = self._split(self.VProj.forward(v))
        O, self.last_node = fused_attn_diff(qp, kp, vp, B * H, Tq, D, 1.0 / math.sqrt(D), causal,
                                            H=H, Sk=Tk)
        ctx = O.reshape(B, H, Tq, D).transpose(0, 2, 1, 3).reshape(B, Tq, self.EmbedDim)
        return self.OutProj.forward(ctx)

    def _fused(self, q, k, v, causal, kv_len, attn_mask=None):
        B, Tq, _ = q.shape
        Tk = k.shape[1]
        H, D = self.NumHeads, self.HeadDim
        qp = self._split(self.QProj.forward(q))
        kp = self._split(self.KProj.forward(k))
        vp = self._split(self.VProj.forward(v))
        scale = 1.0 / math.sqrt(D)
        if Tq == Tk and kv_len is None and attn_mask is None:
            O = fused_attn_f64(qp, kp, vp, B * H, Tq, D, scale, causal)
        else:
            # the wider gate: cross-attention, prefix key padding, additive mask
            O = hip.FlashAttnF64Ex(qp, kp, vp, B, H, Tq, Tk, D, scale, causal, kv_len=kv_len,
                                   attn_mask=attn_mask)
        ctx = O.reshape(B, H, Tq, D).transpose(0, 2, 1, 3).reshape(B, Tq, self.EmbedDim)
        return self.OutProj.forward(ctx)

    def forward_masked(self, q, k, v, causal: bool = False, key_padding_mask=None,
                       attn_mask=None, dropout: float = 0.0):
        """ForwardMasked (nn/attention.go:305-341) on the fused core: causal,
        an additive attn_mask in any of expandAttnMask's shapes, and a (B, Tk)
        key-padding mask (nonzero = ignore the key). A padding mask whose
        padded keys form a suffix of each row (how padded batches look) runs
        as per-sequence key counts; any other is added as -1e30 like
        keyPaddingMaskAdd. Attention dropout (Go's math/rand stream) is not
        fused, and a query row with no unblocked key is not defined (the
        reference always runs ForwardMasked on its CPU path; this library has
        none): both raise ValueError."""
        if dropout:
            raise ValueError("nn: the fused core takes no attention dropout")
        q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
        self._check(q, k, v)
        if not fused_attn_available():
            raise RuntimeError("nn: fused attention requires the HIP library and a gfx950 device")
        kv_len, attn_mask, causal = _core_masks(key_padding_mask, attn_mask, q.shape[0],
                                                self.NumHeads, q.shape[1], k.shape[1], causal)
        return self._fused(q, k, v, causal, kv_len, attn_mask)

    # ---- device-resident forward (new: weights and intermediates in HBM) ----
    def to_device(self) -> "ResidentMultiHeadAttention":
        """This layer with its weights uploaded once: forward / forward_masked
        then run projections, core and output projection on the device with
        one upload and one download per call (gonn_hip_mha_*)."""
        return ResidentMultiHeadAttention(self)

    # ---- incremental decoding (new: the reference has no KV cache) ----
    def new_cache(self, batch: int, max_len: int) -> "hip.KVCache":
        """A device KV cache for this layer: batch sequences, max_len positions."""
        return hip.KVCache(batch, self.NumHeads, max_len, self.HeadDim)

    def forward_incremental(self, x, cache: "hip.KVCache"):
        """Causal self-attention of new tokens x (B, T, E) over the tokens the
        cache holds plus themselves: each new position is projected, its K/V
        appended, and its query attended over the cache (one position at a
        time, so position t sees exactly the positions <= t). Output row t
        equals row (cached + t) of forward_fused(seq, seq, seq, causal=True)
        over the whole sequence (top-left causal mask, nn/attention.go:185-196,
        is what the cache realises)."""
        x = np.asarray(x, dtype=np.float64)
        E = self.EmbedDim
        if x.ndim != 3 or x.shape[2] != E:
            raise ValueError(f"MultiHeadAttention: x shape {x.shape}, want (B, T, {E})")
        B, T, _ = x.shape
        H, D = self.NumHeads, self.HeadDim
        if (cache.B, cache.H, cache.D) != (B, H, D):
            raise ValueError(f"MultiHeadAttention: cache is ({cache.B},{cache.H},*,{cache.D}), "
                             f"want ({B},{H},*,{D})")
        qp = self._split(self.QProj.forward(x))
        kp = self._split(self.KProj.forward(x))
        vp = self._split(self.VProj.forward(x))
        scale = 1.0 / math.sqrt(D)
        ctx = np.empty((B, H, T, D))
        for t in range(T):
            cache.append_f64(kp[:, :, t:t + 1, :], vp[:, :, t:t + 1, :])
            ctx[:, :, t, :] = cache.attend_f64(qp[:, :, t, :], scale)
        ctx = ctx.transpose(0, 2, 1, 3).reshape(B, T, E)
        return self.OutProj.forward(ctx)


def attn_decode(q, kcache, vcache, kv_len, scale=None, split_keys: int = 0):
    """KV-cache decode on device tensors: ForwardMasked with a key-padding mask
    pad[b][t] = (t >= kv_len[b]) on the post-projection core."""
    return hip.attn_decode(q, kcache, vcache, kv_len, scale=scale, split_keys=split_keys)


class ResidentMultiHeadAttention:
    """MultiHeadAttention.forward / forward_masked on a hip.DeviceMHA: the
    same results as the host-projection path (same fp64 GEMM order up to
    rounding of the library GEMM, the same fused core), with the weights and
    every intermediate in HBM."""

    def __init__(self, mha: MultiHeadAttention):
        if not fused_attn_available():
            raise RuntimeError("nn: the resident MHA requires the HIP library and a gfx950 device")
        self._mha = mha
        L = (mha.QProj, mha.KProj, mha.VProj, mha.OutProj)
        self.dev = hip.DeviceMHA(mha.EmbedDim, mha.NumHeads, *[x for l in L for x in (l.W, l.b)])

    def close(self) -> None:
        self.dev.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def forward(self, q, k, v, causal: bool = False):
        same_k, same_v = k is q, v is k
        q = np.asarray(q, dtype=np.float64)
        k = q if same_k else np.asarray(k, dtype=np.float64)
        v = k if same_v else np.asarray(v, dtype=np.float64)
        self._mha._check(q, k, v)
        return self.dev.forward(q, k, v, causal)

    def forward_masked(self, q, k, v, causal: bool = False, key_padding_mask=None,
                       attn_mask=None, dropout: float = 0.0):
        if attn_mask is not None or dropout:
            raise ValueError("nn: the resident layer takes no additive attn mask or dropout "
                             "(MultiHeadAttention.forward_masked takes the mask)")
        same_k, same_v = k is q, v is k
        q = np.asarray(q, dtype=np.float64)
        k = q if same_k else np.asarray(k, dtype=np.float64)
        v = k if same_v else np.asarray(v, dtype=np.float64)
        self._mha._check(q, k, v)
        kv_len = _kv_len_from_mask(key_padding_mask, q.shape[0], k.shape[1])
        return self.dev.forward(q, k, v, causal, kv_len)

    def new_cache(self, batch: int, max_len: int) -> "hip.KVCache":
        """A device KV cache for forward_incremental: batch sequences of up to
        max_len positions, heads at the padded head dim (64 or 128)."""
        dp = 64 if self._mha.HeadDim <= 64 else 128
        return hip.KVCache(batch, self._mha.NumHeads, max_len, dp)

    def forward_incremental(self, x, cache: "hip.KVCache"):
        """MultiHeadAttention.forward_incremental on the device: the T new
        positions of every sequence (x (B, T, E) host fp64) are projected,
        appended and attended in one device pass (the causal multi-token
        attend), with one upload, one download and one host synchronisation
        per call instead of a round trip per position. Output row t equals row
        (cached + t) of the causal forward over the whole sequence."""
        torch = hip._torch()
        x = np.ascontiguousarray(x, dtype=np.float64)
        E = self._mha.EmbedDim
        if x.ndim != 3 or x.shape[2] != E:
            raise ValueError(f"MultiHeadAttention: x shape {x.shape}, want (B, T, {E})")
        out = self.dev.forward_incremental_dev(torch.from_numpy(x).cuda(), cache)
        return out.cpu().numpy()
