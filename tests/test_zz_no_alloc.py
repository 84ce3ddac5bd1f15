"""The allocation-free backward (fa2_bwd_f16_noalloc) through the C ABI: its dQ, dK, dV
equal those of fa2_bwd_f16 with a caller workspace bit for bit, on consecutive calls
that share the library's scratch array (the second with a smaller input, so stale
contents of the first would show), for the split modes 7 and 2 + 4."""
import ctypes

import pytest
import torch

import fa2_capi as capi

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def inputs(B, H, S, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, S, 64, generator=g).half().to(DEV) for _ in range(4)]


def keep_words(lib, B, H, S, causal):
    """A buffer for the forward's dropout keep-bit words (16-byte aligned int32)."""
    n = (lib.fa2_dropout_mask_bytes_causal(B, H, S) if causal else lib.fa2_dropout_mask_bytes(B, H, S)) // 4
    return torch.zeros(n, dtype=torch.int32, device=DEV)


def run_pair(lib, B, H, S, causal, p, seed, words=False):
    """(workspace-entry-point grads, no-alloc grads) for modes 7 and 2+4; with
    `words` the forward writes its keep-bit words and both backwards read them."""
    q, k, v, do = inputs(B, H, S, seed)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=DEV)
    mask = keep_words(lib, B, H, S, causal) if words else None
    pf = capi.fwd_params(q, k, v, o, lse, 0.125, causal=causal, dropout_p=p, seed=seed, mask=mask)
    assert lib.fa2_fwd_f16(ctypes.byref(pf), None) == 0, lib.fa2_last_error()
    ws = torch.full((lib.fa2_bwd_workspace_bytes(B, H, S) // 4,), float("nan"), device=DEV)
    outs = {}
    for name in ("workspace", "noalloc7", "noalloc2+4"):
        dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
        pb = capi.bwd_params(q, k, v, o, lse, do, dq, dk, dv, 0.125, causal=causal, dropout_p=p, seed=seed,
                             mask=mask)
        if name == "workspace":
            rc = lib.fa2_bwd_f16(ctypes.byref(pb), 7, ws.data_ptr(), ws.numel() * 4, None)
            assert rc == 0, lib.fa2_last_error()
        elif name == "noalloc7":
            assert lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 7, None) == 0, lib.fa2_last_error()
        else:
            assert lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 2, None) == 0, lib.fa2_last_error()
            assert lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 4, None) == 0, lib.fa2_last_error()
        outs[name] = (dq, dk, dv)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("causal,p,words", [(True, 0.0, False), (False, 0.0, False), (True, 0.1, False),
                                             (True, 0.1, True), (False, 0.1, True)])
def test_noalloc_backward_equals_workspace_backward(causal, p, words):
    lib = capi.load()
    for B, H, S in ((2, 3, 1000), (1, 2, 300)):      # second call smaller than the first
        say(f"case noalloc B={B} H={H} S={S} causal={causal} p={p} keep-bit words={words}")
        outs = run_pair(lib, B, H, S, causal, p, seed=S + int(causal), words=words)
        ref = outs["workspace"]
        for name in ("noalloc7", "noalloc2+4"):
            for tname, a, b in zip(("dQ", "dK", "dV"), outs[name], ref):
                assert torch.isfinite(a).all(), (name, tname)
                assert torch.equal(a, b), f"{name} {tname} differs (B={B} H={H} S={S})"


def test_noalloc_rejects_oversize_and_bad_mode():
    lib = capi.load()
    assert lib.fa2_bwd_noalloc_scratch_bytes(8, 12, 4096) <= 32 << 20   # benchmark configuration 2 fits
    q = torch.zeros(1, 1, 64, 64, dtype=torch.float16, device=DEV)
    pb = capi.bwd_params(q, q, q, q, torch.zeros(1, 1, 64, device=DEV), q, q, q, q, 0.125)
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 15, None) == 4   # modes are 0..7
    pb.B, pb.H, pb.S = 64, 64, 4096          # 24*B*H*S bytes > 32 MiB, rejected before any launch
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 7, None) == 5
    assert b"FA2_BWD_SCRATCH_MAX_BYTES" in lib.fa2_last_error()


def test_noalloc_backward_under_graph_capture():
    """After one call on the device (which looks up the scratch array's address),
    the allocation-free backward can be captured into a HIP graph: every replay,
    with eager work and synchronisations between replays, equals fa2_bwd_f16
    bit for bit."""
    lib = capi.load()
    B, H, S = 2, 3, 700
    say(f"case noalloc graph capture B={B} H={H} S={S}")
    q, k, v, do = inputs(B, H, S, seed=5)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=DEV)
    pf = capi.fwd_params(q, k, v, o, lse, 0.125)
    assert lib.fa2_fwd_f16(ctypes.byref(pf), None) == 0, lib.fa2_last_error()
    ws = torch.empty(lib.fa2_bwd_workspace_bytes(B, H, S) // 4, device=DEV)
    ref = [torch.empty_like(q) for _ in range(3)]
    pr = capi.bwd_params(q, k, v, o, lse, do, *ref, 0.125)
    assert lib.fa2_bwd_f16(ctypes.byref(pr), 7, ws.data_ptr(), ws.numel() * 4, None) == 0, lib.fa2_last_error()
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    pb = capi.bwd_params(q, k, v, o, lse, do, *got, 0.125)
    assert lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 7, None) == 0, lib.fa2_last_error()   # set-up call
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        rc = lib.fa2_bwd_f16_noalloc(ctypes.byref(pb), 7, ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, lib.fa2_last_error()
    for i in range(3):
        for t in got:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), f"replay {i}: {name} differs"
