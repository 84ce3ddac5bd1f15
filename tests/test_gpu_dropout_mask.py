"""Dropout keep-bit words: the forward stores the keep bit of every pair it
computes, the split backward reads them instead of hashing again.

The words must hold exactly the bits of the dropout hash, so the mask path is
checked bit for bit against the hash path (O, LSE, dQ, dK, dV identical), and
the words themselves against the oracle's keep mask decoded through the
layout include/fa2_mi355x.h documents.  The hash path is pinned against the
oracle by test_gpu_parity.py::test_dropout_vs_oracle."""
import ctypes
import itertools

import numpy as np
import pytest
import torch

import fa2_capi as capi
from oracle import fa2_oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def rand_inputs(B, H, S, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, S, 64, generator=g).half().to(DEV) for _ in range(4)]


def mask_bits(words, B, H, S, causal=False):
    """[B*H, S, S] keep bits (query row, key col) read out of the words through the
    layout include/fa2_mi355x.h documents: bit 31 - (16*kb + 8*hh + e) of the word of
    (tile t, half g, query i) holds key 64*t + 32*kb + 16*hh + 8*(e//4) + 4*g + e%4
    (T = 2*ceil(S/128) tiles, R = S rounded up to 256 queries).  Without the causal mask the
    word is ((bh*T + t)*2 + g)*R + i; with it, tile t keeps queries i >= r = 128*(t//2) in
    runs of n = R - r words, word bh*W(T/2) + W(t//2) + (t%2)*2*n + g*n + (i - r), with
    W(j) = 4*j*R - 256*j*(j-1).  Pairs a causal layout does not hold read as False."""
    T, R = 2 * ((S + 127) // 128), (S + 255) // 256 * 256
    key = np.arange(S)
    t, r = key // 64, key % 64
    kb, hh, e_hi, g, e_lo = r // 32, (r // 16) % 2, (r // 8) % 2, (r // 4) % 2, r % 4
    bit = 31 - (16 * kb + 8 * hh + 4 * e_hi + e_lo)
    row = np.arange(S)[:, None]                          # [S rows, 1]
    if causal:
        W = lambda j: 4 * j * R - 256 * j * (j - 1)
        j, o = t // 2, t % 2
        r0, n = 128 * j, R - 128 * j
        held = row >= r0[None, :]                        # [S rows, S keys]
        idx = np.where(held, W(j) + o * 2 * n + g * n + (row - r0), 0)
        w = words.reshape(B * H, W(T // 2))[:, idx]      # [BH, S rows, S keys]
    else:
        held = np.ones((S, S), bool)
        w = words.reshape(B * H, T * 2 * R)[:, ((t * 2 + g) * R)[None, :] + row]
    bits = ((w >> bit[None, None, :].astype(np.uint32)) & 1).astype(bool)
    return bits & held[None]


SHAPES = [(1, 2, 1), (1, 2, 63), (2, 2, 160), (1, 3, 257), (1, 1, 513), (2, 2, 1000)]


@pytest.mark.parametrize("B,H,S", SHAPES)
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("p", [0.1, 0.5])
def test_mask_path_bitwise_equals_hash_path(fa, B, H, S, causal, p):
    say(f"case mask vs hash B={B} H={H} S={S} causal={causal} p={p}")
    ext = fa.extension()
    q, k, v, do = rand_inputs(B, H, S, seed=S + 7)
    seed = 0x5EED + S
    o, lse = ext.fa_fwd(q, k, v, p, causal, 0.125, seed)
    o2, lse2, mask = ext.fa_fwd_mask(q, k, v, p, causal, 0.125, seed)
    lib = capi.load()
    want_bytes = lib.fa2_dropout_mask_bytes_causal(B, H, S) if causal else lib.fa2_dropout_mask_bytes(B, H, S)
    assert mask.dtype == torch.int32 and mask.numel() * 4 == want_bytes
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    ref = ext.fa_bwd(q, k, v, o, lse, do, p, causal, 0.125, seed, 7)
    got = ext.fa_bwd(q, k, v, o, lse, do, p, causal, 0.125, seed, 7, mask=mask)
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.equal(a, b), f"{name} differs"
    # the dQ pass alone, and the dK/dV pass alone: the binding runs mode 4 as
    # delta kernel + dK/dV, whose delta sums in another order than the dQ
    # pass's, so it is compared with mode 4 without the words
    dq = ext.fa_bwd(q, k, v, o, lse, do, p, causal, 0.125, seed, 2, mask=mask)[0]
    dk, dv = ext.fa_bwd(q, k, v, o, lse, do, p, causal, 0.125, seed, 4, mask=mask)[1:]
    dk4, dv4 = ext.fa_bwd(q, k, v, o, lse, do, p, causal, 0.125, seed, 4)[1:]
    torch.cuda.synchronize()
    assert torch.equal(dq, ref[0]) and torch.equal(dk, dk4) and torch.equal(dv, dv4)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S", [70, 300])
def test_mask_words_match_oracle_keep(fa, causal, S):
    """Through the C ABI into a buffer prefilled with a pattern: every visible
    pair's bit equals the oracle's keep bit (a word the forward skipped would
    keep the pattern and fail)."""
    say(f"case mask words S={S} causal={causal}")
    B, H, p, seed = 2, 2, 0.3, 0xBEEF
    q, k, v, _ = rand_inputs(B, H, S, seed=5)
    lib = capi.load()
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=DEV)
    nbytes = lib.fa2_dropout_mask_bytes_causal(B, H, S) if causal else lib.fa2_dropout_mask_bytes(B, H, S)
    words = torch.full((nbytes // 4,), 0x55555555, dtype=torch.int32, device=DEV)
    prm = capi.fwd_params(q, k, v, o, lse, 0.125, causal=causal, dropout_p=p, seed=seed, mask=words)
    assert lib.fa2_fwd_f16(ctypes.byref(prm), None) == 0, lib.fa2_last_error()
    torch.cuda.synchronize()
    got = mask_bits(words.cpu().numpy().view(np.uint32), B, H, S, causal)
    want = orc.keep_mask(seed, B, H, S, p).reshape(B * H, S, S)
    vis = np.ones((S, S), bool) if not causal else np.tri(S, dtype=bool)
    bad = (got != want) & vis[None]
    assert not bad.any(), f"{int(bad.sum())} keep bits differ, first at {np.argwhere(bad)[0]}"


def test_autograd_mask_on_off_identical(fa, monkeypatch):
    """flash_attn_v100 with dropout: the gradients with the keep-bit words
    (default) equal those of the hash-only backward (mask size cap 0)."""
    say("case autograd mask on/off")
    q0, k0, v0, do = rand_inputs(2, 3, 384, seed=11)
    grads = []
    for cap in (1 << 30, 0):
        monkeypatch.setattr(fa, "DROPOUT_MASK_MAX_BYTES", cap)
        torch.manual_seed(1234)
        monkeypatch.setattr(fa, "_SEED_COUNTER", itertools.count(1))
        q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
        o = fa.flash_attn_v100(q, k, v, dropout_p=0.2, causal=True)
        o.backward(do)
        grads.append([o.detach()] + [t.grad for t in (q, k, v)])
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_words_only_when_a_gradient_follows(fa, monkeypatch):
    """Without a gradient to compute (no_grad, or no input requiring one) the forward stores
    no keep-bit words; with one, the words are saved for the backward."""
    say("case words only with a backward")
    q, k, v, _ = rand_inputs(1, 2, 256, seed=21)
    ext = fa.extension()
    calls = []

    class Spy:
        def __getattr__(self, name):
            fn = getattr(ext, name)
            if name == "fa_fwd_mask":
                def wrapped(*a, **kw):
                    calls.append(name)
                    return fn(*a, **kw)
                return wrapped
            return fn

    monkeypatch.setattr(fa, "_EXT", Spy())
    with torch.no_grad():
        fa.flash_attn_v100(q, k, v, dropout_p=0.2, causal=True)
    fa.flash_attn_v100(q, k, v, dropout_p=0.2, causal=True)        # no input requires grad
    assert calls == []
    qg = q.clone().requires_grad_(True)
    o = fa.flash_attn_v100(qg, k, v, dropout_p=0.2, causal=True)
    assert calls == ["fa_fwd_mask"] and o.grad_fn.saved_tensors[5] is not None
    o.sum().backward()
    torch.cuda.synchronize()


@pytest.mark.parametrize("shape", ["config2", "long"])
def test_full_size_mask_path_bitwise_equals_hash_path(fa, shape):
    """At the benchmark shape (B=8 H=12 S=4096, 201 MB of words) and at S=16384 (B=1 H=2): the word
    path's gradients equal the hash path's bit for bit, so the word addressing holds at full size."""
    import fa2_workloads as wl
    say(f"case full-size mask vs hash {shape}")
    ext = fa.extension()
    if shape == "config2":
        q, k, v, do = wl.config_inputs(2, device=DEV)
    else:
        q, k, v, do = rand_inputs(1, 2, 16384, seed=3)
    p, seed = 0.1, 0xD00D
    o, lse = ext.fa_fwd(q, k, v, p, True, 0.125, seed)
    o2, lse2, mask = ext.fa_fwd_mask(q, k, v, p, True, 0.125, seed)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    ref = ext.fa_bwd(q, k, v, o, lse, do, p, True, 0.125, seed, 7)
    got = ext.fa_bwd(q, k, v, o, lse, do, p, True, 0.125, seed, 7, mask=mask)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.equal(a, b), f"{name} differs"


@pytest.mark.parametrize("use_mask", [False, True])
def test_config2_dropout_bands_vs_oracle(fa, use_mask):
    """Config 2 at full size (B=8 H=12 S=4096, RoPE inputs) with p = 0.1, through the
    hash path and through the keep-bit words: O, LSE, dQ of two 256-row query bands, and
    dK, dV of the last 256 keys (seen only by the last 256 queries), against fp32
    computations from the band's [H, 256, S] score slab with the oracle's keep mask for
    those rows -- P_d = keep * P / (1-p) with LSE from the un-dropped P, dS = P_d * dP - P * delta
    (reference @ None: flash_attn_v100.cu:208-231, flash_attn_v100_bwd.cu:149-191,373-396).
    Bars: O max-abs 2e-3 / (1-p), LSE max-abs 1e-3, gradients relative L2 1e-2."""
    import fa2_workloads as wl
    say(f"case config-2 dropout bands vs oracle, keep-bit words={use_mask}")
    ext = fa.extension()
    q, k, v, do = wl.config_inputs(2, device=DEV)
    B, H, S, _ = q.shape
    p, seed, R, scale = 0.1, 0x5EED5, 256, 0.125
    if use_mask:
        o, lse, mask = ext.fa_fwd_mask(q, k, v, p, True, scale, seed)
        dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do, p, True, scale, seed, 7, mask=mask)
    else:
        o, lse = ext.fa_fwd(q, k, v, p, True, scale, seed)
        dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do, p, True, scale, seed, 7)
    torch.cuda.synchronize()
    rel = lambda a, b: ((a.float() - b).norm() / b.norm()).item()
    cols = torch.arange(S, device=DEV)
    for b in (0, B - 1):
        kf, vf = k[b].float(), v[b].float()                                  # [H, S, 64]
        for r0 in (S // 2 - R // 2, S - R):
            rows = np.arange(r0, r0 + R)
            keep = orc.dropout_keep(seed, rows[None, :, None], np.arange(S)[None, None, :],
                                    (b * H + np.arange(H))[:, None, None], p)   # [H, R, S]
            keep = torch.from_numpy(keep).to(DEV).float()
            s = torch.matmul(q[b, :, r0:r0 + R].float(), kf.transpose(-1, -2).contiguous()) * scale
            s.masked_fill_(cols.view(1, -1) > torch.arange(r0, r0 + R, device=DEV).view(-1, 1), float("-inf"))
            rl = torch.logsumexp(s, dim=-1)
            pr = torch.exp(s - rl.unsqueeze(-1))
            pd = pr * keep / (1 - p)
            ro = torch.matmul(pd, vf)
            dob = do[b, :, r0:r0 + R].float()
            delta = (ro * dob).sum(-1, keepdim=True)
            dpm = torch.matmul(dob, vf.transpose(-1, -2).contiguous())
            ds = pd * dpm - pr * delta
            rdq = torch.matmul(ds, kf) * scale
            eo = (o[b, :, r0:r0 + R].float() - ro).abs().max().item()
            el = (lse[b, :, r0:r0 + R] - rl).abs().max().item()
            eq = rel(dq[b, :, r0:r0 + R], rdq)
            say(f"b={b} rows {r0}..{r0 + R - 1}: O maxabs {eo:.2e}  LSE maxabs {el:.2e}  dQ rel {eq:.2e}  "
                f"kept {keep[:, :, :r0 + 1].mean().item():.4f}")
            assert eo <= 2e-3 / (1 - p) and el <= 1e-3 and eq <= 1e-2
            if r0 == S - R:
                qb = q[b, :, r0:].float()
                rdv = torch.matmul(pd[:, :, r0:].transpose(-1, -2).contiguous(), dob)
                rdk = torch.matmul(ds[:, :, r0:].transpose(-1, -2).contiguous(), qb) * scale
                edv, edk = rel(dv[b, :, r0:], rdv), rel(dk[b, :, r0:], rdk)
                say(f"b={b} last {R} keys: dK rel {edk:.2e}  dV rel {edv:.2e}")
                assert edk <= 1e-2 and edv <= 1e-2
