"""GPU parity of the gfx950 kernels (run on the MI355X box).

Bars (from the benchmark definition): O max-abs <= 2e-3 against the
reference's own path (SDPA math in fp32/fp64 on the same fp16 inputs), and
dQ/dK/dV relative error <= 1e-2 (relative L2 norm; max-abs is printed too).
Small shapes are checked against the fp64 CPU oracle and the committed golden
fixtures; the benchmark's full shapes are checked on sampled heads against
SDPA math in fp32 on the GPU plus size-independent properties.
"""
import ctypes
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

import fa2_capi as capi
import fa2_workloads as wl
from oracle import fa2_oracle as orc

pytestmark = pytest.mark.gpu

O_TOL = 2e-3
G_TOL = 1e-2
LSE_TOL = 1e-3
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fa2_golden.npz")


def say(*a):
    print(*a, flush=True)


def run_kernel(fa, q, k, v, do, causal=True, scale=0.125, p=0.0, seed=0, mode=7):
    """fa_bwd `mode`: the reference's bit mask (1 delta, 2 dQ, 4 dK/dV; 7 = all)."""
    ext = fa.extension()
    o, lse = ext.fa_fwd(q, k, v, p, causal, scale, seed)
    dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do, p, causal, scale, seed, mode)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


def check_against(name, got, ref, o_tol=O_TOL):
    o, lse, dq, dk, dv = (t.detach().float().cpu().numpy() for t in got)
    ro, rlse, rdq, rdk, rdv = (np.asarray(x, np.float64) for x in ref)
    eo = orc.max_abs(o, ro)
    el = orc.max_abs(lse, rlse)
    eg = [orc.rel_l2(a, b) for a, b in ((dq, rdq), (dk, rdk), (dv, rdv))]
    ma = [orc.max_abs(a, b) for a, b in ((dq, rdq), (dk, rdk), (dv, rdv))]
    say(f"{name}: O maxabs {eo:.2e}  LSE maxabs {el:.2e}  rel dQ/dK/dV {eg[0]:.2e} {eg[1]:.2e} {eg[2]:.2e}"
        f"  maxabs {ma[0]:.2e} {ma[1]:.2e} {ma[2]:.2e}")
    assert eo <= o_tol, f"{name}: O max-abs {eo}"
    assert el <= LSE_TOL, f"{name}: LSE max-abs {el}"
    for e, n in zip(eg, ("dQ", "dK", "dV")):
        assert e <= G_TOL, f"{name}: {n} rel err {e}"


def oracle_ref(q, k, v, do, causal, scale, p=0.0, seed=0):
    qn, kn, vn, don = (t.detach().float().cpu().numpy() for t in (q, k, v, do))
    keep = orc.keep_mask(seed, q.shape[0], q.shape[1], q.shape[2], p) if p > 0 else None
    o, lse = orc.attention_dense_fwd(qn, kn, vn, causal=causal, scale=scale, keep=keep, p=p)
    dq, dk, dv, _ = orc.attention_bwd(qn, kn, vn, o, lse, don, causal=causal, scale=scale, keep=keep, p=p)
    return o, lse, dq, dk, dv


def sdpa_ref_gpu(q, k, v, do, causal=True, scale=0.125):
    """The reference's fallback path (SDPA, MATH backend) in fp32 on the GPU."""
    tq, tk, tv = (t.detach().float().contiguous().requires_grad_(True) for t in (q, k, v))
    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=scale)
    o.backward(do.float().contiguous())
    s = torch.matmul(tq.detach(), tk.detach().transpose(-1, -2).contiguous()) * scale
    if causal:
        S = q.shape[-2]
        s.masked_fill_(torch.ones(S, S, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    return [t.detach().double().cpu().numpy() for t in (o, lse, tq.grad, tk.grad, tv.grad)]


def rand_inputs(B, H, S, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(B, H, S, 64, generator=g) * scale).half().to(DEV) for _ in range(4)]


@pytest.mark.parametrize("S", [1, 2, 17, 63, 64, 65, 127, 129, 200, 256, 257, 300, 513])
@pytest.mark.parametrize("causal", [True, False])
def test_small_shapes_vs_oracle(fa, S, causal):
    say(f"case small S={S} causal={causal}")
    q, k, v, do = rand_inputs(1, 2, S, seed=S + 1000 * causal)
    got = run_kernel(fa, q, k, v, do, causal=causal)
    check_against(f"S={S} causal={causal}", got, oracle_ref(q, k, v, do, causal, 0.125))


def test_golden_fixtures(fa):
    z = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in z.files if not k.startswith("mask")})
    for name in names:
        B, H, S, causal, scale, p, seed = z[f"{name}/meta"]
        say(f"case golden {name}")
        q, k, v, do = (torch.from_numpy(z[f"{name}/{t}"]).to(DEV) for t in ("q", "k", "v", "do"))
        got = run_kernel(fa, q, k, v, do, causal=bool(causal), scale=float(scale), p=float(p), seed=int(seed))
        ref = [z[f"{name}/{t}"] for t in ("o", "lse", "dq", "dk", "dv")]
        check_against(f"golden {name}", got, ref, o_tol=O_TOL / (1.0 - float(p)))


@pytest.mark.parametrize("scale", [0.3, -0.2, 0.0, 0.05])
def test_softmax_scales(fa, scale):
    say(f"case scale={scale}")
    q, k, v, do = rand_inputs(1, 2, 190, seed=77)
    got = run_kernel(fa, q, k, v, do, scale=scale)
    check_against(f"scale={scale}", got, oracle_ref(q, k, v, do, True, scale))


@pytest.mark.parametrize("scale,amp,S", [(1.0, 4.0, 97), (0.125, 4.0, 250), (1e-3, 1.0, 130), (1e-25, 1.0, 70)])
def test_row_term_extremes(fa, scale, amp, S):
    """Large logits (LSE up to ~10^2 in log2 units, so -LSE*log2e/scale2 is large) and tiny scales:
    without dropout the dK/dV pass starts its S and dP chains at the row terms -LSE*log2e/scale2 and
    -delta for scale2 >= 1e-20, and subtracts them per element below that (the 1e-25 case); S not a
    multiple of 32 exercises the last term block."""
    say(f"case row terms scale={scale} amp={amp} S={S}")
    q, k, v, do = rand_inputs(1, 2, S, seed=31)
    q, k = (q.float() * amp).half(), (k.float() * amp).half()
    got = run_kernel(fa, q, k, v, do, scale=scale)
    ref = oracle_ref(q, k, v, do, True, scale)
    if scale >= 1e-6:
        check_against(f"row terms scale={scale} amp={amp}", got, ref)
        return
    # dQ and dK carry the factor scale (~1e-25): below fp16's range, they are zero in fp16 output
    # like any fp16 kernel's; O, LSE and dV do not depend on it.
    o, lse, dv = (got[i].float().cpu().numpy() for i in (0, 1, 4))
    assert orc.max_abs(o, np.asarray(ref[0])) <= O_TOL
    assert orc.max_abs(lse, np.asarray(ref[1])) <= LSE_TOL
    assert orc.rel_l2(dv, np.asarray(ref[4], np.float64)) <= G_TOL


@pytest.mark.parametrize("S", [160, 1100])
def test_subnormal_output_gradient(fa, S):
    """dO of order 1e-4, so that about half its fp16 values are subnormal: delta = rowsum(O * dO) and
    everything downstream must keep them (a flush to zero would bias delta and every dS); S = 1100
    takes the two-block dQ pass, S = 160 the narrow one."""
    say(f"case subnormal dO S={S}")
    q, k, v, do = rand_inputs(1, 2, S, seed=23)
    do = (do.float() * 1e-4).half()
    assert (do.abs() < 2.0 ** -14).float().mean().item() > 0.3
    got = run_kernel(fa, q, k, v, do)
    check_against(f"subnormal dO S={S}", got, oracle_ref(q, k, v, do, True, 0.125))


@pytest.mark.parametrize("p,seed", [(0.1, 1), (0.5, 0xC0FFEE), (0.9, 42)])
def test_dropout_vs_oracle(fa, p, seed):
    say(f"case dropout p={p} seed={seed}")
    q, k, v, do = rand_inputs(2, 2, 160, seed=seed % 1000)
    got = run_kernel(fa, q, k, v, do, p=p, seed=seed)
    # Dropout scales O by 1/(1-p); the fp16 output's own rounding scales with
    # it, so the O bar does too (grads keep the relative bar).
    check_against(f"dropout p={p}", got, oracle_ref(q, k, v, do, True, 0.125, p=p, seed=seed),
                  o_tol=O_TOL / (1.0 - p))


@pytest.mark.parametrize("scale,causal", [(0.125, True), (1.0, True), (-0.3, False), (1.0, False)])
def test_dropout_scales(fa, scale, causal):
    """Dropout at the scales the other dropout tests leave out (1.0, where scale*log2(e) > 1, and a
    negative one, which negates an operand), causal and not: with the forward's keep-bit words and
    with the hash, against the oracle, and the two bitwise equal."""
    p, seed = 0.1, 0xD0
    say(f"case dropout scale={scale} causal={causal}")
    ext = fa.extension()
    q, k, v, do = rand_inputs(1, 2, 190, seed=19)
    o, lse, mask = ext.fa_fwd_mask(q, k, v, p, causal, scale, seed)
    words = ext.fa_bwd(q, k, v, o, lse, do, p, causal, scale, seed, 7, mask=mask)
    hashed = ext.fa_bwd(q, k, v, o, lse, do, p, causal, scale, seed, 7)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), words, hashed):
        assert torch.equal(a, b), f"{name}: keep words and hash differ"
    check_against(f"dropout scale={scale} causal={causal}", (o, lse, *words),
                  oracle_ref(q, k, v, do, causal, scale, p=p, seed=seed), o_tol=O_TOL / (1.0 - p))


def test_medium_vs_sdpa_math_gpu(fa):
    say("case medium B=2 H=4 S=1024 vs SDPA math fp32")
    q, k, v, do = rand_inputs(2, 4, 1024, seed=5)
    got = run_kernel(fa, q, k, v, do)
    check_against("medium", got, sdpa_ref_gpu(q, k, v, do))


def test_train_py_layouts_are_bitwise_identical(fa):
    """q/k as dense [B,S,H,D] views, v a view of the fused qkv tensor, dO the
    transposed view of a [B,S,H,D] grad: same bits as contiguous inputs."""
    say("case train.py layouts")
    B, S, H = 2, 333, 12
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(B, S, 3 * H * 64, generator=g).half().to(DEV)
    q, k, v = qkv.chunk(3, dim=-1)
    q = q.view(B, S, H, 64).transpose(1, 2)
    k = k.contiguous().view(B, S, H, 64).transpose(1, 2)
    v = v.view(B, S, H, 64).transpose(1, 2)
    do = torch.randn(B, S, H, 64, generator=g).half().to(DEV).transpose(1, 2)
    assert v.stride(2) == 3 * H * 64 and not do.is_contiguous()
    got = run_kernel(fa, q, k, v, do)
    ref = run_kernel(fa, *(t.contiguous() for t in (q, k, v, do)))
    for a, b, n in zip(got, ref, ("o", "lse", "dq", "dk", "dv")):
        assert torch.equal(a, b), n


def test_autograd_wrapper_and_sdpa_shim(fa):
    say("case autograd wrapper")
    q, k, v, do = rand_inputs(1, 3, 300, seed=11)
    qs, ks, vs = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = fa.flash_attn_v100(qs, ks, vs)
    out.backward(do)
    got = run_kernel(fa, q, k, v, do)
    assert torch.equal(out.detach(), got[0])
    for a, b in zip((qs.grad, ks.grad, vs.grad), got[2:]):
        assert torch.equal(a, b)
    shim = fa.sdpa(q, k, v, is_causal=True)
    assert torch.equal(shim, got[0])
    masked = fa.sdpa(q.float(), k.float(), v.float(), is_causal=True)   # fp32 -> SDPA fallback
    assert masked.dtype == torch.float32


def test_capi_direct_matches_binding(fa):
    """Call fa2_fwd_f16 / fa2_bwd_f16 through ctypes on torch's current stream."""
    say("case C ABI direct")
    lib = capi.load()
    q, k, v, do = rand_inputs(2, 3, 200, seed=21)
    B, H, S, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = capi.fwd_params(q, k, v, o, lse, 0.125)
    assert lib.fa2_fwd_f16(ctypes.byref(p), stream) == 0, lib.fa2_last_error()
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    ws = torch.empty(lib.fa2_bwd_workspace_bytes(B, H, S) // 4, device=DEV)
    assert ws.numel() * 4 >= B * H * S * 8 + B * H * ((S + 31) // 32 * 32) * 8   # delta, LSE*log2e, row terms
    pb = capi.bwd_params(q, k, v, o, lse, do, dq, dk, dv, 0.125)
    assert lib.fa2_bwd_f16(ctypes.byref(pb), 7, ws.data_ptr(), ws.numel() * 4, stream) == 0
    torch.cuda.synchronize()
    ref = run_kernel(fa, q, k, v, do)
    for a, b in zip((o, lse, dq, dk, dv), ref):
        assert torch.equal(a, b)
    # delta left in the workspace equals rowsum(O * dO)
    delta = (o.float() * do.float()).sum(-1).reshape(-1)
    assert torch.allclose(ws[: B * H * S], delta, atol=1e-3, rtol=1e-3)


def test_capi_outputs_with_4_element_row_strides(fa):
    """O, dQ, dK, dV written through the C ABI into padded buffers whose row stride (68 elements) is a
    multiple of 4 but not of 8 -- accepted by the ABI, and the output stores' 8-byte path: the same bits
    as the binding's contiguous outputs, and the padding (NaN) untouched."""
    say("case C ABI outputs with 68-element rows")
    lib = capi.load()
    q, k, v, do = rand_inputs(2, 3, 200, seed=23)
    B, H, S, _ = q.shape
    bufs = [torch.full((B, H, S, 68), float("nan"), dtype=torch.float16, device=DEV) for _ in range(4)]
    o, dq, dk, dv = (t[..., :64] for t in bufs)
    assert o.stride(2) == 68 and o.data_ptr() % 16 == 0
    lse = torch.empty(B, H, S, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = capi.fwd_params(q, k, v, o, lse, 0.125)
    assert lib.fa2_fwd_f16(ctypes.byref(p), stream) == 0, lib.fa2_last_error()
    ws = torch.empty(lib.fa2_bwd_workspace_bytes(B, H, S) // 4, device=DEV)
    # O is an input of the backward, whose rows the ABI wants 16-byte aligned: a contiguous copy.
    pb = capi.bwd_params(q, k, v, o.contiguous(), lse, do, dq, dk, dv, 0.125)
    assert lib.fa2_bwd_f16(ctypes.byref(pb), 7, ws.data_ptr(), ws.numel() * 4, stream) == 0, lib.fa2_last_error()
    torch.cuda.synchronize()
    ref = run_kernel(fa, q, k, v, do)
    for name, got, want in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv), ref):
        assert torch.equal(got, want), name
    for name, t in zip(("o", "dq", "dk", "dv"), bufs):
        assert torch.isnan(t[..., 64:]).all(), f"{name}: padding written"


def test_empty_inputs(fa):
    """Empty batch / sequence: outputs of the right (empty) shapes, no launch, no error."""
    say("case empty inputs")
    ext = fa.extension()
    for shape in ((0, 2, 16, 64), (2, 3, 0, 64)):
        q, k, v, do = (torch.empty(shape, dtype=torch.float16, device=DEV) for _ in range(4))
        o, lse = ext.fa_fwd(q, k, v, 0.0, True, 0.125, 0)
        assert o.shape == q.shape and lse.shape == q.shape[:3]
        dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do, 0.0, True, 0.125, 0, 7)
        assert dq.shape == dk.shape == dv.shape == q.shape
        kk = torch.empty(shape[0], shape[1], 5, 64, dtype=torch.float16, device=DEV)
        o2, lse2 = ext.fa_fwd_kv(q, kk, kk, True, 0.125, 0)
        assert o2.shape == q.shape and lse2.shape == q.shape[:3]
    torch.cuda.synchronize()


def test_capi_split_modes(fa):
    """dQ (mode 2) then dK/dV (mode 4) as two calls sharing one workspace give the bits of mode 7;
    delta-only (mode 1) then mode 4 matches the oracle (its delta sums in another order)."""
    say("case C ABI split modes")
    lib = capi.load()
    q, k, v, do = rand_inputs(1, 2, 231, seed=23)
    B, H, S, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    pf = capi.fwd_params(q, k, v, o, lse, 0.125)
    assert lib.fa2_fwd_f16(ctypes.byref(pf), stream) == 0, lib.fa2_last_error()
    nbytes = lib.fa2_bwd_workspace_bytes(B, H, S)
    outs = {}
    for name, modes in (("7", (7,)), ("2+4", (2, 4)), ("1+4", (1, 4))):
        ws = torch.full((nbytes // 4,), float("nan"), device=DEV)   # nothing may be read unwritten
        dq, dk, dv = (torch.zeros_like(q) for _ in range(3))
        pb = capi.bwd_params(q, k, v, o, lse, do, dq, dk, dv, 0.125)
        for m in modes:
            assert lib.fa2_bwd_f16(ctypes.byref(pb), m, ws.data_ptr(), ws.numel() * 4, stream) == 0, \
                lib.fa2_last_error()
        torch.cuda.synchronize()
        outs[name] = (dq, dk, dv)
    for a, b in zip(outs["7"][1:], outs["2+4"][1:]):
        assert torch.equal(a, b)
    assert torch.equal(outs["7"][0], outs["2+4"][0])
    ref = oracle_ref(q, k, v, do, True, 0.125)
    for got, want, n in zip(outs["1+4"][1:], ref[3:], ("dK", "dV")):
        e = orc.rel_l2(got.float().cpu().numpy(), np.asarray(want, np.float64))
        assert e <= G_TOL, f"mode 1+4 {n} rel err {e}"


def test_deterministic(fa):
    """The forward and the backward are run-to-run identical, and fa_bwd, like
    the reference's, reads only bits 1, 2 and 4 of `mode` (mode 15 = mode 7)."""
    say("case determinism")
    q, k, v, do = rand_inputs(2, 4, 777, seed=3)
    a = run_kernel(fa, q, k, v, do, mode=7)
    b = run_kernel(fa, q, k, v, do, mode=7)
    c = run_kernel(fa, q, k, v, do, mode=15)
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(x, z)


def _check_sampled_heads(fa, name, q, k, v, do, heads):
    got = run_kernel(fa, q, k, v, do)
    o, lse, dq, dk, dv = got
    for t in got:
        assert torch.isfinite(t).all(), name
    # p = 0: rows of P sum to 1, so the dV rows sum to the dO rows per head.
    sdv = dv.float().sum(dim=2)
    sdo = do.float().sum(dim=2)
    err = (sdv - sdo).abs().max().item() / max(1.0, sdo.abs().max().item())
    say(f"{name}: sum-rows(dV) vs sum-rows(dO) rel {err:.2e}")
    assert err < 1e-2
    for b, h in heads:
        sl = lambda t: t[b:b + 1, h:h + 1]
        ref = sdpa_ref_gpu(sl(q), sl(k), sl(v), sl(do))
        check_against(f"{name} b={b} h={h}", [sl(t) for t in got], ref)


def test_config2_full_shape(fa):
    say("case config 2 full shape B=8 H=12 S=4096 (RoPE inputs)")
    q, k, v, do = wl.config_inputs(2, device=DEV)
    _check_sampled_heads(fa, "config2", q, k, v, do, [(0, 0), (7, 11), (3, 5)])


@pytest.mark.parametrize("S", [512, 1024, 2048, 4096])
def test_config3_buckets(fa, S):
    say(f"case config 3 S={S}")
    q, k, v, do = wl.config_inputs(f"3-{S}", device=DEV)
    _check_sampled_heads(fa, f"config3-{S}", q, k, v, do, [(0, 0), (q.shape[0] - 1, 11)])


@pytest.mark.parametrize("B,H,S", [(64, 12, 512), (26, 16, 512), (26, 16, 1024), (31, 12, 1050), (2, 4, 300),
                                   (1024, 8, 128), (3, 5, 2100)])
def test_every_head_written_and_correct(fa, B, H, S):
    """Short sequences with B*H a multiple of 8 run the forward and dQ pass in groups of 16 heads per
    XCD (the last group smaller when B*H/8 is not a multiple of 16: 26*16/8 = 52 heads; one head per
    XCD at B*H = 8); B*H = 372 keeps the plain order; 8192 heads of one 128-query block each give the
    largest grids; B*H = 15 at S = 2100 takes the pipelined forward and the two-block dQ pass.  Outputs
    start as NaN and every head of every output must be written and match SDPA MATH fp32 on the GPU."""
    say(f"case every head B={B} H={H} S={S}")
    lib = capi.load()
    q, k, v, do = rand_inputs(B, H, S, seed=S + H)
    o, dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(4))
    lse = torch.full((B, H, S), float("nan"), device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    pf = capi.fwd_params(q, k, v, o, lse, 0.125)
    assert lib.fa2_fwd_f16(ctypes.byref(pf), stream) == 0, lib.fa2_last_error()
    ws = torch.full((lib.fa2_bwd_workspace_bytes(B, H, S) // 4,), float("nan"), device=DEV)
    pb = capi.bwd_params(q, k, v, o, lse, do, dq, dk, dv, 0.125)
    assert lib.fa2_bwd_f16(ctypes.byref(pb), 7, ws.data_ptr(), ws.numel() * 4, stream) == 0, lib.fa2_last_error()
    torch.cuda.synchronize()
    for name, t in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv)):
        assert torch.isfinite(t).all(), f"{name}: unwritten or non-finite entries"
    ro, rlse, rdq, rdk, rdv = (torch.from_numpy(x) for x in sdpa_ref_gpu(q, k, v, do))
    eo = (o.double().cpu() - ro).abs().amax(dim=(2, 3))          # per head
    el = (lse.double().cpu() - rlse).abs().amax(dim=2)
    say(f"every head: O max-abs {eo.max().item():.2e}, LSE max-abs {el.max().item():.2e}")
    assert eo.max().item() <= O_TOL and el.max().item() <= LSE_TOL
    for name, got, want in (("dQ", dq, rdq), ("dK", dk, rdk), ("dV", dv, rdv)):
        g = got.double().cpu()
        e = ((g - want).norm(dim=(2, 3)) / want.norm(dim=(2, 3)).clamp_min(1e-30))   # per head
        say(f"every head: {name} rel (worst head) {e.max().item():.2e}")
        assert e.max().item() <= G_TOL, name


def test_config4_outlier_rows(fa):
    say("case config 4 B=8 H=16 S=4096 with x8 rows")
    q, k, v, do = wl.config_inputs(4, device=DEV)
    norms = q.float().norm(dim=-1)                       # [B,H,S]
    b, h = divmod(int(norms.amax(dim=2).flatten().argmax()), q.shape[1])  # head holding the largest row
    _check_sampled_heads(fa, "config4", q, k, v, do, [(b, h), (0, 0)])


def test_rope_bitwise_vs_oracle(fa):
    say("case rope fwd/bwd bitwise")
    B, S, H = 2, 257, 12
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(B, S, 3 * H * 64, generator=g).half()
    q, k, _ = qkv.chunk(3, dim=-1)
    q = q.view(B, S, H, 64).transpose(1, 2)
    k = k.view(B, S, H, 64).transpose(1, 2)
    cos, sin = wl.rope_tables(S)
    cos_pad = torch.zeros(S, 128)
    cos_pad[:, :64] = cos                     # row-padded view like cos_cached[..., :64]
    sin_pad = torch.zeros(S, 128)
    sin_pad[:, :64] = sin
    c2, s2 = cos_pad.to(DEV)[:, :64], sin_pad.to(DEV)[:, :64]
    qd, kd = q.to(DEV), k.to(DEV)
    assert fa.rope_can_use(qd, kd, c2, s2)
    qo, ko = fa.rope(qd, kd, c2, s2)
    torch.cuda.synchronize()
    for got, x in ((qo, q), (ko, k)):
        ref = orc.rope_fwd(x.numpy(), cos.numpy(), sin.numpy())
        assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16))
    gq = torch.randn(B, H, S, 64, generator=g).half()
    gk = torch.randn(B, H, S, 64, generator=g).half()
    dq, dk = fa.extension().rope_bwd(gq.to(DEV), gk.to(DEV), c2, s2, qd, kd)
    torch.cuda.synchronize()
    for got, gg in ((dq, gq), (dk, gk)):
        ref = orc.rope_bwd(gg.numpy(), cos.numpy(), sin.numpy())
        assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_rope_scalar_path_bitwise(fa):
    """Rows only 4-byte aligned (base offset by two halves, strides not multiples of 8):
    the C ABI takes the scalar RoPE kernel; forward and backward still bitwise equal to
    the oracle."""
    say("case rope scalar path (4-byte aligned rows)")
    B, S, H = 2, 100, 3
    g = torch.Generator().manual_seed(6)
    buf = torch.randn(B, S, H, 66, generator=g).half()
    q = buf[..., 2:].transpose(1, 2)                           # (B,H,S,64), base +4 bytes, stride 66
    kbuf = torch.randn(B, S, H, 66, generator=g).half()
    k = kbuf[..., 2:].transpose(1, 2)
    cos, sin = wl.rope_tables(S)
    qd, kd = buf.to(DEV)[..., 2:].transpose(1, 2), kbuf.to(DEV)[..., 2:].transpose(1, 2)
    assert qd.data_ptr() % 16 == 4 and qd.stride(1) % 8 != 0
    ext = fa.extension()
    qo, ko = ext.rope_fwd(qd, kd, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    for got, x in ((qo, q), (ko, k)):
        ref = orc.rope_fwd(x.contiguous().numpy(), cos.numpy(), sin.numpy())
        assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16))
    dq, dk = ext.rope_bwd(qd, kd, cos.to(DEV), sin.to(DEV), qd, kd)
    torch.cuda.synchronize()
    for got, x in ((dq, q), (dk, k)):
        ref = orc.rope_bwd(x.contiguous().numpy(), cos.numpy(), sin.numpy())
        assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("layout", ["fused_qkv", "bhsd"])
def test_rope_config2_shape_bitwise(fa, layout):
    """The vector RoPE kernel at config-2 shape (B=8 H=12 S=4096) in train.py's fused-qkv
    layout and in contiguous (B,H,S,D): bitwise equal to the eager fp32 expression."""
    say(f"case rope config-2 shape {layout}")
    B, S, H = 8, 4096, 12
    g = torch.Generator().manual_seed(7)
    if layout == "fused_qkv":
        qkv = torch.randn(B, S, 3 * H * 64, generator=g).half().to(DEV)
        q, k, _ = (t.view(B, S, H, 64).transpose(1, 2) for t in qkv.chunk(3, dim=-1))
    else:
        q, k = (torch.randn(B, H, S, 64, generator=g).half().to(DEV) for _ in range(2))
    cos, sin = (t.to(DEV) for t in wl.rope_tables(S))
    qo, ko = fa.extension().rope_fwd(q, k, cos, sin)
    c, s_ = cos[None, None], sin[None, None]
    rot = lambda x: torch.cat((-x[..., 32:], x[..., :32]), dim=-1)
    for got, x in ((qo, q), (ko, k)):
        ref = (x.float() * c + rot(x.float()) * s_).half()
        assert torch.equal(got, ref)

