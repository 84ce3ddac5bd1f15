"""Synthetic inputs for the benchmark configurations of the attention path.

Every tensor is drawn in fp32 from ``torch.Generator('cpu').manual_seed(seed)``
(machine independent), in the order Q, K, V, dO, in the [B, S, H, D] memory
layout train.py produces (``qkv.view(B, S, H, D)``), then cast and moved to the
device and presented as [B, H, S, D] through ``.transpose(1, 2)``.

Configurations (the ``configs`` list of the benchmark definition):
  1  B=2  H=4  S=256  D=64 fp32, N(0,1)                        (CPU fallback case)
  2  B=8  H=12 S=4096 D=64 fp16, Q/K/V N(0,1)*0.5 with RoPE on Q and K
     (base 10000, inv_freq over d_model 768, first 64 columns), dO N(0,1)
  3  S in {512,1024,2048,4096}, B=32768/S, H=12, fp16, N(0,1)
  4  B=8  H=16 S=4096 fp16, N(0,1), ceil(1%) of the (b,s,h) Q rows scaled x8
     (rows chosen by a seeded permutation)
"""

import math

import torch

HEAD_DIM = 64


def rope_tables(seq_len, d_model=768, head_dim=HEAD_DIM, base=10000.0):
    """cos/sin [S, head_dim] fp32 as train.py builds them (train.py:1877-1906):
    inv_freq = base^(-arange(0, d_model, 2)/d_model), emb = cat(freqs, freqs),
    truncated to the head dim -- so cos[:, d] != cos[:, d+32]."""
    inv_freq = 1.0 / (base ** (torch.arange(0, d_model, 2).float() / d_model))
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos()[:, :head_dim].contiguous(), emb.sin()[:, :head_dim].contiguous()


def apply_rope_bshd(x, cos, sin):
    """x [B,S,H,D] fp32; out = x*cos + rotate_half(x)*sin (train.py:1898-1918)."""
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    x1, x2 = x.chunk(2, dim=-1)
    rot = torch.cat((-x2, x1), dim=-1)
    return x * c + rot * s


def make_inputs(B, H, S, seed=0, dtype=torch.float16, device="cpu", scale=1.0, rope=False,
                outlier_frac=0.0, requires_grad=False):
    """Q, K, V, dO as [B,H,S,64] views of [B,S,H,64] storage."""
    g = torch.Generator("cpu").manual_seed(seed)
    shape = (B, S, H, HEAD_DIM)
    q = torch.randn(shape, generator=g) * scale
    k = torch.randn(shape, generator=g) * scale
    v = torch.randn(shape, generator=g) * scale
    do = torch.randn(shape, generator=g)
    if rope:
        cos, sin = rope_tables(S)
        q = apply_rope_bshd(q, cos, sin)
        k = apply_rope_bshd(k, cos, sin)
    if outlier_frac > 0:
        n_rows = B * S * H
        n_out = math.ceil(outlier_frac * n_rows)
        idx = torch.randperm(n_rows, generator=g)[:n_out]
        flat = q.view(n_rows, HEAD_DIM)
        flat[idx] *= 8.0
    out = []
    for t in (q, k, v, do):
        t = t.to(dtype).to(device).transpose(1, 2)
        if requires_grad and t is not None:
            t.requires_grad_(True)
        out.append(t)
    return tuple(out)


CONFIGS = {
    1: dict(B=2, H=4, S=256, dtype=torch.float32, scale=1.0, rope=False, outlier_frac=0.0),
    2: dict(B=8, H=12, S=4096, dtype=torch.float16, scale=0.5, rope=True, outlier_frac=0.0),
    "3-512": dict(B=64, H=12, S=512, dtype=torch.float16, scale=1.0, rope=False, outlier_frac=0.0),
    "3-1024": dict(B=32, H=12, S=1024, dtype=torch.float16, scale=1.0, rope=False, outlier_frac=0.0),
    "3-2048": dict(B=16, H=12, S=2048, dtype=torch.float16, scale=1.0, rope=False, outlier_frac=0.0),
    "3-4096": dict(B=8, H=12, S=4096, dtype=torch.float16, scale=1.0, rope=False, outlier_frac=0.0),
    4: dict(B=8, H=16, S=4096, dtype=torch.float16, scale=1.0, rope=False, outlier_frac=0.01),
}


def config_inputs(name, seed=0, device="cpu", **overrides):
    cfg = dict(CONFIGS[name])
    cfg.update(overrides)
    return make_inputs(cfg["B"], cfg["H"], cfg["S"], seed=seed, dtype=cfg["dtype"], device=device,
                       scale=cfg["scale"], rope=cfg["rope"], outlier_frac=cfg["outlier_frac"])


def causal_flops(B, H, S, D=HEAD_DIM):
    """Algorithmic flops (causal-halved convention): fwd 2*B*H*S^2*D, bwd 5*B*H*S^2*D."""
    unit = B * H * S * S * D
    return 2 * unit, 5 * unit


def causal_bytes(B, H, S, D=HEAD_DIM, elem=2):
    """Compulsory HBM bytes of fwd+bwd: 12 fp16 tensor passes + 2 fp32 LSE passes."""
    return 12 * B * H * S * D * elem + 2 * B * H * S * 4
