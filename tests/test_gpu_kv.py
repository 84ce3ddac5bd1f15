"""GPU parity of the key/value-length forward (fa2_fwd_kv_f16: prefill chunks
against a KV cache, decode) and of the inference routing in ``sdpa()``.

Bars as for the square forward: O max-abs <= 2e-3 and LSE max-abs <= 1e-3
against the fp64 CPU oracle (pinned for these shapes in tests/test_oracle.py)
or torch SDPA in fp32 on the GPU; the square case is bitwise equal to fa_fwd.
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fa2_capi as capi
from oracle import fa2_oracle as orc

pytestmark = pytest.mark.gpu

O_TOL = 2e-3
LSE_TOL = 1e-3
DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def inputs(B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, 64, generator=g).half().to(DEV)
    k, v = (torch.randn(B, H, Sk, 64, generator=g).half().to(DEV) for _ in range(2))
    return q, k, v


def check(name, o, lse, q, k, v, causal, coff, scale=0.125):
    ro, rl = orc.attention_dense_fwd(*(t.float().cpu().numpy() for t in (q, k, v)), causal=causal,
                                     scale=scale, causal_offset=coff)
    o, lse = o.float().cpu().numpy(), lse.float().cpu().numpy()
    seen = np.isfinite(rl)
    eo = orc.max_abs(o, ro)
    el = orc.max_abs(lse[seen], rl[seen]) if seen.any() else 0.0
    say(f"{name}: O maxabs {eo:.2e}  LSE maxabs {el:.2e}  rows seeing no key {int((~seen).sum())}")
    assert eo <= O_TOL, f"{name}: O max-abs {eo}"
    assert el <= LSE_TOL, f"{name}: LSE max-abs {el}"
    assert np.all(lse[~seen] == -np.inf), f"{name}: LSE of rows that see no key"


@pytest.mark.parametrize("Sq,Sk,causal,coff", [
    (1, 300, False, 0),        # decode: one query, every cached key
    (1, 300, True, 299),       # decode as a bottom-right causal chunk (same visibility)
    (37, 300, True, 263),      # prefill chunk, bottom-right
    (64, 256, True, 192),      # chunk and cache on tile boundaries
    (130, 70, True, 0),        # SDPA is_causal alignment with S_q > S_k (top-left)
    (50, 20, True, -30),       # bottom-right with S_q > S_k: the first 30 queries see nothing
    (100, 333, False, 0),      # non-causal, non-square
    (200, 129, True, 5),       # an offset that is no multiple of the tiles
])
@pytest.mark.parametrize("nsplit", [1, 3, 0])
def test_kv_forward_vs_oracle(fa, Sq, Sk, causal, coff, nsplit):
    """nsplit 1: one pass; 3: three key slices merged; 0: the binding's automatic choice."""
    say(f"case kv Sq={Sq} Sk={Sk} causal={causal} offset={coff} nsplit={nsplit}")
    q, k, v = inputs(2, 3, Sq, Sk, seed=Sq * 7 + Sk)
    o, lse = fa.extension().fa_fwd_kv(q, k, v, causal, 0.125, coff, nsplit)
    torch.cuda.synchronize()
    check(f"kv Sq={Sq} Sk={Sk} c={causal} off={coff} split={nsplit}", o, lse, q, k, v, causal, coff)


@pytest.mark.parametrize("nsplit", [2, 5, 16, 40])
def test_kv_split_matches_single_pass(fa, nsplit):
    """Slices merged agree with one pass to rounding (O to fp16, LSE to a few fp32 ulps of values
    up to ~20, summed in another order), also with more slices than the causal range of some query
    blocks reaches and with empty trailing slices (40 > 26 tiles)."""
    say(f"case kv split={nsplit} vs single pass")
    q, k, v = inputs(2, 2, 300, 1650, seed=nsplit)
    ext = fa.extension()
    for causal, coff in ((True, 1350), (True, 0), (False, 0)):
        o1, l1 = ext.fa_fwd_kv(q, k, v, causal, 0.125, coff, 1)
        o2, l2 = ext.fa_fwd_kv(q, k, v, causal, 0.125, coff, nsplit)
        torch.cuda.synchronize()
        eo = (o1.float() - o2.float()).abs().max().item()
        el = (l1 - l2).abs().max().item()
        say(f"split {nsplit} causal={causal} off={coff}: O {eo:.2e} LSE {el:.2e}")
        assert eo <= 2e-3 and el <= 5e-4


@pytest.mark.parametrize("causal", [True, False])
def test_kv_square_is_fa_fwd_bitwise(fa, causal):
    say(f"case kv square causal={causal}")
    q, k, v = inputs(2, 2, 333, 333, seed=5)
    ext = fa.extension()
    o1, l1 = ext.fa_fwd_kv(q, k, v, causal, 0.125, 0, 1)     # one pass (no key slices)
    o2, l2 = ext.fa_fwd(q, k, v, 0.0, causal, 0.125, 0)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_kvcache_chunk_matches_tail_of_square(fa):
    """The bottom-right chunk of the last S_q queries against all S_k keys reproduces the last rows
    of the square causal forward (what a KV cache must do), to fp16 rounding."""
    say("case kvcache chunk = tail of square")
    B, H, Sk, Sq = 2, 4, 1000, 200
    qf, k, v = inputs(B, H, Sk, Sk, seed=9)
    full, _ = fa.extension().fa_fwd(qf, k, v, 0.0, True, 0.125, 0)
    chunk = fa.flash_attn_kvcache(qf[:, :, Sk - Sq:], k, v)
    err = (chunk.float() - full[:, :, Sk - Sq:].float()).abs().max().item()
    say(f"chunk vs square tail: max-abs {err:.2e}")
    assert err <= 1e-3


def test_sdpa_routes_inference_shapes(fa):
    """Decode and non-square causal calls without a gradient reach the kernel (bitwise equal to
    fa_fwd_kv) and agree with torch SDPA in fp32; a call that needs a gradient stays on SDPA."""
    say("case sdpa inference routing")
    ext = fa.extension()
    for Sq, Sk, causal in ((1, 777, False), (48, 500, True), (64, 64, False)):
        q, k, v = inputs(1, 6, Sq, Sk, seed=Sq + Sk)
        with torch.no_grad():
            got = fa.sdpa(q, k, v, is_causal=causal)
        want, _ = ext.fa_fwd_kv(q, k, v, causal, 64 ** -0.5, 0)
        assert torch.equal(got, want), (Sq, Sk, causal)
        ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal)
        err = (got.float() - ref).abs().max().item()
        say(f"sdpa Sq={Sq} Sk={Sk} causal={causal}: max-abs vs SDPA fp32 {err:.2e}")
        assert err <= O_TOL
    q, k, v = inputs(1, 2, 16, 40, seed=1)
    q.requires_grad_(True)
    out = fa.sdpa(q, k, v, is_causal=False)       # needs a gradient: SDPA path, differentiable
    out.float().sum().backward()
    assert q.grad is not None


def test_capi_kv_split_entry_point(fa):
    """fa2_fwd_kv_split_f16 through ctypes, on a NaN-filled workspace (every partial it reads must
    be written), equals the binding with the same nsplit."""
    say("case C ABI fa2_fwd_kv_split_f16")
    lib = capi.load()
    q, k, v = inputs(1, 3, 1, 900, seed=4)
    B, H, Sq, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, H, Sq, device=DEV)
    p = capi.fwd_params(q, k, v, o, lse, 0.125, causal=False)
    nbytes = lib.fa2_fwd_kv_workspace_bytes(B, H, Sq, 7)
    assert nbytes == 7 * B * H * Sq * 66 * 4
    ws = torch.full((nbytes // 4,), float("nan"), device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.fa2_fwd_kv_split_f16(ctypes.byref(p), 900, 0, 7, ws.data_ptr(), nbytes, stream) == 0, \
        lib.fa2_last_error()
    assert lib.fa2_fwd_kv_split_f16(ctypes.byref(p), 900, 0, 7, ws.data_ptr(), nbytes - 4, stream) == 5
    torch.cuda.synchronize()
    o2, l2 = fa.extension().fa_fwd_kv(q, k, v, False, 0.125, 0, 7)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, l2)
    check("capi split", o, lse, q, k, v, False, 0)


def test_capi_kv_entry_point(fa):
    """fa2_fwd_kv_f16 through ctypes on torch's stream equals the binding."""
    say("case C ABI fa2_fwd_kv_f16")
    lib = capi.load()
    q, k, v = inputs(1, 2, 40, 170, seed=3)
    B, H, Sq, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, H, Sq, device=DEV)
    p = capi.fwd_params(q, k, v, o, lse, 0.125, causal=True)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.fa2_fwd_kv_f16(ctypes.byref(p), 170, 130, stream) == 0, lib.fa2_last_error()
    torch.cuda.synchronize()
    o2, l2 = fa.extension().fa_fwd_kv(q, k, v, True, 0.125, 130)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, l2)
