"""Minimal pre-norm decoder in the reference's shape, used to exercise the
attention path inside a full training step (benchmark configuration 5) and in
the model-level drop-in test.

It mirrors what reaches the attention kernel in the reference
(reference @ None: train.py:1861-2105) -- fused QKV projection, q/k/v as
(B,S,H,D) views transposed to (B,H,S,D), fused RoPE through
``flash_attn_v100_cuda.rope`` (eager fallback otherwise), attention through
``flash_attn_v100_cuda.flash_attn_v100`` (SDPA fallback otherwise),
``attn.transpose(1,2).contiguous().view(B,S,D)`` and the output projection --
plus RMSNorm, a SwiGLU FFN and a tied LM head.  It is a consumer of the path,
not a reimplementation of the reference's training runtime.
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

import fa2_workloads as wl


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


class Attention(nn.Module):
    def __init__(self, d_model, n_heads, fa=None, use_kernel=True):
        super().__init__()
        self.h, self.d = n_heads, d_model // n_heads
        self.wqkv = nn.Linear(d_model, 3 * d_model, bias=False)
        self.wo = nn.Linear(d_model, d_model, bias=False)
        self.fa, self.use_kernel = fa, use_kernel
        self.attn_fn = None  # optional override (q, k, v) -> o, used for timing
        # Fallback path only: attention through SDPA's math backend in fp32 (the
        # reference path the kernel's parity is defined against), cast back.
        self.ref_fp32 = False

    def forward(self, x, cos, sin):
        B, S, D = x.shape
        q, k, v = self.wqkv(x).chunk(3, dim=-1)
        q = q.view(B, S, self.h, self.d).transpose(1, 2)
        k = k.view(B, S, self.h, self.d).transpose(1, 2)
        v = v.view(B, S, self.h, self.d).transpose(1, 2)
        fa = self.fa if self.use_kernel else None
        if fa is not None and fa.rope_can_use(q, k, cos, sin):
            q, k = fa.rope(q, k, cos, sin)
        else:
            c, s = cos[None, None], sin[None, None]
            q, k = q * c + rotate_half(q) * s, k * c + rotate_half(k) * s
        if torch.is_autocast_enabled():
            q, k, v = (t.half() if t.dtype == torch.float32 else t for t in (q, k, v))
        if fa is not None and fa.can_use(q, k, v):
            attn = self.attn_fn(q, k, v) if self.attn_fn else fa.flash_attn_v100(q, k, v, causal=True)
        elif self.ref_fp32:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            with torch.autocast(x.device.type, enabled=False), sdpa_kernel(SDPBackend.MATH):
                attn = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True).to(q.dtype)
        else:
            attn = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.wo(attn.transpose(1, 2).contiguous().view(B, S, D))

    def forward_cached(self, x, cos, sin, cache):
        """Inference: x holds the last S_new positions of the sequence, cos/sin
        their RoPE rows, and cache = [k, v] the earlier positions' rotated keys
        and values ((B,H,S_past,64) each, or None), extended in place.  The
        queries see every cached key and the causal part of their own: the
        bottom-right mask an HF-style KV-cache decoder builds
        (reference @ None: hf_template/modeling_universal_lm.py:228-251),
        through ``flash_attn_kvcache`` or, on the fallback path, SDPA with
        that mask spelled out."""
        B, S, D = x.shape
        q, k, v = (t.view(B, S, self.h, self.d).transpose(1, 2) for t in self.wqkv(x).chunk(3, dim=-1))
        fa = self.fa if self.use_kernel else None
        if fa is not None and fa.rope_can_use(q, k, cos, sin):
            q, k = fa.rope(q, k, cos, sin)
        else:
            c, s = cos[None, None], sin[None, None]
            q, k = ((t * c + rotate_half(t) * s).to(v.dtype) for t in (q, k))
        if cache[0] is not None:
            k, v = torch.cat([cache[0], k], dim=2), torch.cat([cache[1], v], dim=2)
        cache[0], cache[1] = k, v
        if fa is not None:
            attn = fa.flash_attn_kvcache(q, k, v, causal=True)
        else:
            Sk = k.shape[2]
            mask = torch.ones(S, Sk, dtype=torch.bool, device=x.device).tril(Sk - S)
            attn = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        return self.wo(attn.transpose(1, 2).contiguous().view(B, S, D))


class Block(nn.Module):
    def __init__(self, d_model, n_heads, d_ff, fa, use_kernel):
        super().__init__()
        self.n1 = nn.RMSNorm(d_model, eps=1e-6)
        self.n2 = nn.RMSNorm(d_model, eps=1e-6)
        self.attn = Attention(d_model, n_heads, fa, use_kernel)
        self.w1 = nn.Linear(d_model, d_ff, bias=False)
        self.w3 = nn.Linear(d_model, d_ff, bias=False)
        self.w2 = nn.Linear(d_ff, d_model, bias=False)

    def forward(self, x, cos, sin):
        x = x + self.attn(self.n1(x), cos, sin)
        h = self.n2(x)
        return x + self.w2(F.silu(self.w1(h)) * self.w3(h))

    def forward_cached(self, x, cos, sin, cache):
        x = x + self.attn.forward_cached(self.n1(x), cos, sin, cache)
        h = self.n2(x)
        return x + self.w2(F.silu(self.w1(h)) * self.w3(h))


class Decoder(nn.Module):
    def __init__(self, vocab=32000, d_model=768, n_heads=12, n_layers=10, d_ff=2048, fa=None, use_kernel=True):
        super().__init__()
        self.emb = nn.Embedding(vocab, d_model)
        self.layers = nn.ModuleList(Block(d_model, n_heads, d_ff, fa, use_kernel) for _ in range(n_layers))
        self.norm = nn.RMSNorm(d_model, eps=1e-6)
        self.head_dim = d_model // n_heads
        self.d_model = d_model
        for p in self.parameters():  # std 0.02 init (train.py:2015-2022)
            nn.init.normal_(p, std=0.02) if p.dim() > 1 else nn.init.ones_(p)

    def forward(self, ids):
        S = ids.shape[1]
        cos, sin = wl.rope_tables(S, d_model=self.d_model, head_dim=self.head_dim)
        cos, sin = cos.to(ids.device), sin.to(ids.device)
        x = self.emb(ids)
        for layer in self.layers:
            x = layer(x, cos, sin)
        return F.linear(self.norm(x), self.emb.weight)  # tied head

    def new_cache(self):
        return [[None, None] for _ in self.layers]

    def forward_cached(self, ids, cache, max_len):
        """Logits of the S_new tokens ``ids`` that follow the positions held in
        ``cache`` (from ``new_cache()``, extended in place): a prefill chunk or
        one decode step.  ``max_len`` sizes the RoPE tables."""
        past = 0 if cache[0][0] is None else cache[0][0].shape[2]
        S = ids.shape[1]
        cos, sin = wl.rope_tables(max_len, d_model=self.d_model, head_dim=self.head_dim)
        cos, sin = (t[past:past + S].contiguous().to(ids.device) for t in (cos, sin))
        x = self.emb(ids)
        for layer, c in zip(self.layers, cache):
            x = layer.forward_cached(x, cos, sin, c)
        return F.linear(self.norm(x), self.emb.weight)

    def loss(self, ids):
        logits = self.forward(ids[:, :-1])
        return F.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), ids[:, 1:].reshape(-1))


def compare_training_step(fa, B, S, n_layers=10, d_ff=2048, vocab=32000, seed=0, device="cuda"):
    """One fp16-autocast training step (GradScaler-scaled backward, then unscaled
    gradients) of the same random-init weights through the kernel path
    (``flash_attn_v100`` + fused ``rope``) and through the reference path (eager
    RoPE, attention by SDPA's math backend in fp32), as train.py's loop runs it
    (reference @ None: train.py:1931-1964, 2341-2424).  Returns (loss_kernel,
    loss_reference, {parameter name: relative L2 error of its gradient})."""
    torch.manual_seed(seed)
    mk = Decoder(vocab=vocab, n_layers=n_layers, d_ff=d_ff, fa=fa, use_kernel=True).to(device)
    mr = Decoder(vocab=vocab, n_layers=n_layers, d_ff=d_ff, fa=None, use_kernel=False).to(device)
    mr.load_state_dict(mk.state_dict())
    for layer in mr.layers:
        layer.attn.ref_fp32 = True
    ids = synthetic_ids(B, S, vocab=vocab, seed=seed + 1, device=device)
    losses = []
    for m in (mk, mr):
        opt = torch.optim.SGD(m.parameters(), lr=0.0)
        scaler = torch.amp.GradScaler(device, init_scale=2.0 ** 16)
        with torch.autocast(device, dtype=torch.float16):
            loss = m.loss(ids)
        scaler.scale(loss).backward()
        scaler.unscale_(opt)
        losses.append(loss.item())
    errs = {}
    for (n, pk), (_, pr) in zip(mk.named_parameters(), mr.named_parameters()):
        errs[n] = ((pk.grad.float() - pr.grad.float()).norm() / pr.grad.float().norm()).item()
    del mk, mr
    return losses[0], losses[1], errs


def synthetic_ids(B, S, vocab=32000, seed=0, device="cpu"):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randint(0, vocab, (B, S + 1), generator=g).to(device)


def step_flops_attention(B, S, H=12, D=64, n_layers=10):
    f, b = wl.causal_flops(B, H, S, D)
    return n_layers * (f + b)


def approx_step_flops(B, S, d_model=768, d_ff=2048, n_layers=10, vocab=32000):
    """6 * params_active * tokens for the linear layers and head, plus attention."""
    lin = n_layers * (4 * d_model * d_model + 3 * d_model * d_ff) + vocab * d_model
    return 6 * lin * B * S + step_flops_attention(B, S, d_model // 64, 64, n_layers)

