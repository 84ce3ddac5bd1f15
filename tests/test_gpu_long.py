"""GPU parity at long sequence lengths, where no dense reference of the whole
problem fits: S = 65536 causal and S = 32768 non-causal for fa_fwd/fa_bwd, and
a 262144-key cache for the inference forward.

What pins the results without the full S x S matrices:
  * causal prefix: rows i < P of O, LSE and dQ depend only on keys <= i, and
    the kernels visit those keys in the same tile order whatever S is, so the
    first P rows equal a run on the length-P prefix bit for bit;
  * explicit fp32 rows: O, LSE and dQ of a band of R query rows from their
    [R, S] score slab, and (causal) dK, dV of the last R keys, which only the
    last R queries see;
  * size-independent sums (p = 0): rows of P sum to 1, so the column sums of
    dV equal those of dO, and rows of dS sum to 0, so the column sums of dK
    vanish.
Bars as elsewhere: O max-abs <= 2e-3, LSE max-abs <= 1e-3, gradients
relative L2 <= 1e-2.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

O_TOL = 2e-3
LSE_TOL = 1e-3
G_TOL = 1e-2
DEV = "cuda"
SCALE = 0.125


def say(*a):
    print(*a, flush=True)


def inputs(H, S, seed, n=4):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(1, H, S, 64, generator=g).half().to(DEV) for _ in range(n)]


def rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def band_reference(q, k, v, do, r0, r1, causal):
    """fp32 O, LSE, dQ of query rows r0..r1-1 and the band's P, dS slabs [H, R, S]."""
    S = k.shape[2]
    qb = q[0, :, r0:r1].float()                                   # [H, R, 64]
    kf, vf = k[0].float(), v[0].float()                           # [H, S, 64]
    s = torch.matmul(qb, kf.transpose(-1, -2).contiguous()) * SCALE   # [H, R, S]
    if causal:
        rows = torch.arange(r0, r1, device=DEV).view(-1, 1)
        cols = torch.arange(S, device=DEV).view(1, -1)
        s.masked_fill_(cols > rows, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                              # [H, R]
    p = torch.exp(s - lse.unsqueeze(-1))
    o = torch.matmul(p, vf)                                       # [H, R, 64]
    dob = do[0, :, r0:r1].float()
    delta = (o * dob).sum(-1, keepdim=True)
    dp = torch.matmul(dob, vf.transpose(-1, -2).contiguous())
    ds = p * (dp - delta)
    dq = torch.matmul(ds, kf) * SCALE
    return o, lse, dq, p, ds


def check_band(name, got, ref, r0, r1):
    o, lse, dq = got[0][0, :, r0:r1], got[1][0, :, r0:r1], got[2][0, :, r0:r1]
    ro, rl, rdq = ref[:3]
    eo = (o.float() - ro).abs().max().item()
    el = (lse.float() - rl).abs().max().item()
    eq = rel(dq, rdq)
    say(f"{name} rows {r0}..{r1 - 1}: O maxabs {eo:.2e}  LSE maxabs {el:.2e}  dQ rel {eq:.2e}")
    assert eo <= O_TOL and el <= LSE_TOL and eq <= G_TOL, name


def check_sums(name, do, dk, dv):
    """Per head: sum_j dV_j = sum_i dO_i and sum_j dK_j = 0 (p = 0), relative
    to the Frobenius norm of dV, dK."""
    for h in range(dv.shape[1]):
        sdv = dv[0, h].float().sum(0)
        sdo = do[0, h].float().sum(0)
        sdk = dk[0, h].float().sum(0)
        ev = ((sdv - sdo).norm() / dv[0, h].float().norm()).item()
        ek = (sdk.norm() / dk[0, h].float().norm()).item()
        say(f"{name} head {h}: |sum dV - sum dO| / |dV| {ev:.2e}   |sum dK| / |dK| {ek:.2e}")
        assert ev <= G_TOL and ek <= G_TOL, name


def test_long_causal_65536(fa):
    S, H, P, R = 65536, 2, 4096, 256
    say(f"case long causal S={S} H={H}")
    q, k, v, do = inputs(H, S, seed=65536)
    ext = fa.extension()
    o, lse = ext.fa_fwd(q, k, v, 0.0, True, SCALE, 0)
    dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do, 0.0, True, SCALE, 0, 7)
    torch.cuda.synchronize()
    for t in (o, lse, dq, dk, dv):
        assert torch.isfinite(t).all()

    say(f"prefix P={P}")
    pq, pk, pv, pdo = (t[:, :, :P] for t in (q, k, v, do))
    po, plse = ext.fa_fwd(pq, pk, pv, 0.0, True, SCALE, 0)
    pdq, _, _ = ext.fa_bwd(pq, pk, pv, po, plse, pdo, 0.0, True, SCALE, 0, 7)
    torch.cuda.synchronize()
    assert torch.equal(o[:, :, :P], po), "O prefix"
    assert torch.equal(lse[:, :, :P], plse), "LSE prefix"
    assert torch.equal(dq[:, :, :P], pdq), "dQ prefix"

    got = (o, lse, dq)
    for r0 in (S // 2 - R // 2, S - R):
        ref = band_reference(q, k, v, do, r0, r0 + R, causal=True)
        check_band("long causal", got, ref, r0, r0 + R)
    # Keys S-R..S-1 are seen only by queries S-R..S-1: their dK, dV follow
    # from the last band's P and dS.
    _, _, _, p, ds = band_reference(q, k, v, do, S - R, S, causal=True)
    qb, dob = q[0, :, S - R:].float(), do[0, :, S - R:].float()
    rdv = torch.matmul(p[:, :, S - R:].transpose(-1, -2).contiguous(), dob)
    rdk = torch.matmul(ds[:, :, S - R:].transpose(-1, -2).contiguous(), qb) * SCALE
    edv, edk = rel(dv[0, :, S - R:], rdv), rel(dk[0, :, S - R:], rdk)
    say(f"long causal last {R} keys: dK rel {edk:.2e}  dV rel {edv:.2e}")
    assert edk <= G_TOL and edv <= G_TOL
    check_sums("long causal", do, dk, dv)


def test_long_noncausal_32768(fa):
    S, H, R = 32768, 1, 256
    say(f"case long non-causal S={S} H={H}")
    q, k, v, do = inputs(H, S, seed=32768)
    ext = fa.extension()
    o, lse = ext.fa_fwd(q, k, v, 0.0, False, SCALE, 0)
    dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do, 0.0, False, SCALE, 0, 7)
    torch.cuda.synchronize()
    for t in (o, lse, dq, dk, dv):
        assert torch.isfinite(t).all()
    for r0 in (0, S - R):
        ref = band_reference(q, k, v, do, r0, r0 + R, causal=False)
        check_band("long non-causal", (o, lse, dq), ref, r0, r0 + R)
    check_sums("long non-causal", do, dk, dv)


@pytest.mark.parametrize("Sq,Sk,causal,coff", [
    (1, 262144, False, 0),          # decode against a 256 Ki-key cache
    (300, 100000, True, 99700),     # prefill chunk at the end of a long cache (bottom-right)
])
def test_long_cache_kv_forward(fa, Sq, Sk, causal, coff):
    H = 4 if Sq == 1 else 2
    say(f"case long cache Sq={Sq} Sk={Sk} causal={causal} offset={coff}")
    g = torch.Generator().manual_seed(Sk)
    q = torch.randn(1, H, Sq, 64, generator=g).half().to(DEV)
    k, v = (torch.randn(1, H, Sk, 64, generator=g).half().to(DEV) for _ in range(2))
    o, lse = fa.extension().fa_fwd_kv(q, k, v, causal, SCALE, coff, 0)
    torch.cuda.synchronize()
    s = torch.matmul(q[0].float(), k[0].float().transpose(-1, -2).contiguous()) * SCALE   # [H, Sq, Sk]
    if causal:
        rows = torch.arange(Sq, device=DEV).view(-1, 1)
        cols = torch.arange(Sk, device=DEV).view(1, -1)
        s.masked_fill_(cols > rows + coff, float("-inf"))
    rl = torch.logsumexp(s, dim=-1)
    ro = torch.matmul(torch.exp(s - rl.unsqueeze(-1)), v[0].float())
    eo = (o[0].float() - ro).abs().max().item()
    el = (lse[0] - rl).abs().max().item()
    say(f"long cache Sq={Sq} Sk={Sk}: O maxabs {eo:.2e}  LSE maxabs {el:.2e}")
    assert eo <= O_TOL and el <= LSE_TOL
