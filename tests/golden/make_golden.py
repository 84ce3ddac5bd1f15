"""Writes tests/golden/fa2_golden.npz: small seeded cases with expected outputs.

The reference ships no golden vectors for this path, so these come from:
  * torch SDPA (MATH backend, fp64) + autograd on the fp16-rounded inputs for
    the p = 0 cases (a library routine, not reference code);
  * the pinned CPU oracle for the dropout cases (hash-mask dropout has no
    library equivalent), together with packed keep-mask bits of the
    reference's hash for a few (seed, bh) 64x64 blocks.
Re-run with `python tests/golden/make_golden.py`; the output is deterministic.
"""
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import fa2_oracle as orc  # noqa: E402

CASES = [  # name, B, H, S, causal, scale, dropout_p, seed
    ("c130", 1, 1, 130, True, 0.125, 0.0, 0),
    ("n65", 1, 1, 65, False, 0.125, 0.0, 0),
    ("c64s", 2, 1, 64, True, -0.3, 0.0, 0),
    ("d96", 1, 1, 96, True, 0.125, 0.2, 1234),
    ("d150", 1, 1, 150, True, 0.125, 0.5, 987654321),
]


def main():
    out = {}
    for i, (name, B, H, S, causal, scale, p, seed) in enumerate(CASES):
        g = torch.Generator().manual_seed(100 + i)
        q, k, v, do = (torch.randn(B, H, S, 64, generator=g).half() for _ in range(4))
        out[f"{name}/q"], out[f"{name}/k"], out[f"{name}/v"], out[f"{name}/do"] = (
            t.numpy() for t in (q, k, v, do))
        out[f"{name}/meta"] = np.array([B, H, S, int(causal), scale, p, seed], dtype=np.float64)
        if p == 0.0:
            tq, tk, tv = (t.double().requires_grad_(True) for t in (q, k, v))
            with sdpa_kernel(SDPBackend.MATH):
                o = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=scale)
            o.backward(do.double())
            _, lse = orc.attention_dense_fwd(q.numpy(), k.numpy(), v.numpy(), causal=causal, scale=scale)
            res = dict(o=o.detach().numpy(), lse=lse, dq=tq.grad.numpy(), dk=tk.grad.numpy(), dv=tv.grad.numpy())
        else:
            keep = orc.keep_mask(seed, B, H, S, p)
            o, lse = orc.attention_dense_fwd(q.numpy(), k.numpy(), v.numpy(), causal=causal, scale=scale,
                                             keep=keep, p=p)
            dq, dk, dv, _ = orc.attention_bwd(q.numpy(), k.numpy(), v.numpy(), o, lse, do.numpy(), causal=causal,
                                              scale=scale, keep=keep, p=p)
            res = dict(o=o, lse=lse, dq=dq, dk=dk, dv=dv)
            out[f"{name}/keepbits"] = np.packbits(keep.reshape(-1))
        for key, val in res.items():
            out[f"{name}/{key}"] = np.asarray(val, np.float32)
    for seed, bh in ((0, 0), (1, 5), (0xDEADBEEF, 95)):
        rows = np.arange(64).reshape(64, 1)
        cols = np.arange(64).reshape(1, 64)
        out[f"mask/{seed}/{bh}"] = np.packbits(orc.dropout_keep(seed, rows, cols, bh, 0.1).reshape(-1))
    np.savez_compressed(os.path.join(HERE, "fa2_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "fa2_golden.npz"))


if __name__ == "__main__":
    main()
