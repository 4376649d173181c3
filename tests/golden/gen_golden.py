"""Generate tests/golden/attn_golden.npz: seeded inputs and expected outputs.

Expected values come from an implementation independent of the oracle:
torch float64 on the CPU (F.scaled_dot_product_attention with an explicit
additive mask built like causalMaskAdd / keyPaddingMaskAdd of
nn/attention.go:185-196, :261-272, torch.logsumexp, and torch autograd for
the gradients of loss = sum(O * dO), the loss of benchmark/flashbwd/main.go:32-38).

    python tests/golden/gen_golden.py
"""
import math
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attn_golden.npz")
CASES = [  # name, BH, Sq, Sk, D, causal, with kv_len
    ("tiny_c", 1, 1, 1, 8, True, False),
    ("s7_nc", 2, 7, 7, 8, False, False),
    ("s7_c", 2, 7, 7, 8, True, False),
    ("s24_c_d64", 1, 24, 24, 64, True, False),
    ("s12_nc_d64", 1, 12, 12, 64, False, False),
    ("cross_c", 2, 5, 9, 16, True, False),
    ("cross_nc", 2, 9, 5, 16, False, False),
    ("pad", 4, 6, 11, 16, False, True),
]


def mask_add(Sq, Sk, causal, kv_len, BH, H):
    m = torch.zeros(BH, Sq, Sk, dtype=torch.float64)
    if causal:
        i = torch.arange(Sq)[:, None]
        j = torch.arange(Sk)[None, :]
        m = m + torch.where(j > i, -1e30, 0.0).to(torch.float64)
    if kv_len is not None:
        for bh in range(BH):
            m[bh, :, kv_len[bh // H]:] += -1e30
    return m


def main():
    out = {}
    for idx, (name, BH, Sq, Sk, D, causal, pad) in enumerate(CASES):
        rng = np.random.default_rng(1000 + idx)
        q, k, v, g = (rng.standard_normal((BH, n, D)) for n in (Sq, Sk, Sk, Sq))
        H = 2 if pad else 1
        kv_len = rng.integers(1, Sk + 1, BH // H).astype(np.int32) if pad else None
        tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
        scale = 1.0 / math.sqrt(D)
        s = (tq @ tk.transpose(1, 2)) * scale + mask_add(Sq, Sk, causal, kv_len, BH, H)
        o = torch.softmax(s, dim=-1) @ tv
        lse = torch.logsumexp(s, dim=-1)
        (o * torch.tensor(g)).sum().backward()
        pre = name + "/"
        out.update({pre + "q": q, pre + "k": k, pre + "v": v, pre + "dO": g,
                    pre + "O": o.detach().numpy(), pre + "LSE": lse.detach().numpy(),
                    pre + "dQ": tq.grad.numpy(), pre + "dK": tk.grad.numpy(),
                    pre + "dV": tv.grad.numpy(),
                    pre + "meta": np.array([BH, Sq, Sk, D, int(causal), H], np.int64)})
        if kv_len is not None:
            out[pre + "kv_len"] = kv_len
    np.savez_compressed(OUT, **out)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
