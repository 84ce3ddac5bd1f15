"""Pins the CPU oracle (oracle/fa2_oracle.py) before any GPU result is trusted.

Each check is independent of the oracle's own formulas: torch's SDPA MATH
backend and autograd (library routines), closed forms, invariants, and an
independent integer evaluation of the dropout hash.  A mistake planted in a
copy of the oracle (dropped delta term, wrong scale placement) is shown to
fail the invariant checks.
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from oracle import fa2_oracle as orc

TAIL_SIZES = [1, 2, 17, 63, 64, 65, 127, 129, 200]


def _rand(shape, seed, scale=1.0):
    g = np.random.default_rng(seed)
    return g.standard_normal(shape) * scale


def _sdpa_math(q, k, v, causal, scale=None):
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale)


def _lse_ref(q, k, causal, scale):
    s = torch.einsum("bhid,bhjd->bhij", q, k) * scale
    if causal:
        S = q.shape[-2]
        s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    return torch.logsumexp(s, dim=-1)


@pytest.mark.parametrize("S", TAIL_SIZES)
@pytest.mark.parametrize("causal", [True, False])
def test_dense_fwd_matches_sdpa_math(S, causal):
    q, k, v = (_rand((1, 2, S, 64), 10 * S + i) for i in range(3))
    o, lse = orc.attention_dense_fwd(q, k, v, causal=causal)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    ref = _sdpa_math(tq, tk, tv, causal).numpy()
    assert orc.max_abs(o, ref) < 1e-12
    assert orc.max_abs(lse, _lse_ref(tq, tk, causal, 0.125).numpy()) < 1e-12


@pytest.mark.parametrize("S", TAIL_SIZES)
def test_tiled_fwd_matches_dense(S):
    q, k, v = (_rand((1, 2, S, 64), 7 * S + i, 2.0) for i in range(3))
    for causal in (True, False):
        o1, l1 = orc.attention_dense_fwd(q, k, v, causal=causal)
        o2, l2 = orc.attention_tiled_fwd(q, k, v, causal=causal)
        assert orc.max_abs(o1, o2) < 1e-11
        assert orc.max_abs(l1, l2) < 1e-11


def test_tiled_fwd_dropout_matches_dense():
    S, p, seed = 150, 0.3, 12345
    q, k, v = (_rand((2, 2, S, 64), 99 + i) for i in range(3))
    keep = orc.keep_mask(seed, 2, 2, S, p)
    o1, l1 = orc.attention_dense_fwd(q, k, v, keep=keep, p=p)
    o2, l2 = orc.attention_tiled_fwd(q, k, v, keep=keep, p=p)
    assert orc.max_abs(o1, o2) < 1e-11
    assert orc.max_abs(l1, l2) < 1e-11


def test_closed_forms():
    S = 130
    q, k, v = (_rand((1, 1, S, 64), 3 + i) for i in range(3))
    # Causal row 0 sees only key 0: O_0 = V_0 exactly.
    o, lse = orc.attention_dense_fwd(q, k, v)
    assert orc.max_abs(o[0, 0, 0], v[0, 0, 0]) < 1e-15
    # Q == 0: uniform weights, O_i = mean(V_0..V_i), LSE_i = ln(i+1).
    o, lse = orc.attention_tiled_fwd(np.zeros_like(q), k, v)
    cum = np.cumsum(v[0, 0], axis=0) / np.arange(1, S + 1)[:, None]
    assert orc.max_abs(o[0, 0], cum) < 1e-12
    assert orc.max_abs(lse[0, 0], np.log(np.arange(1, S + 1))) < 1e-12
    # LSE_i >= max_j s_ij (visible j).
    o, lse = orc.attention_dense_fwd(q, k, v)
    s = np.einsum("id,jd->ij", q[0, 0], k[0, 0]) * 0.125
    s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    assert np.all(lse[0, 0] >= s.max(axis=1) - 1e-12)


@pytest.mark.parametrize("S", [1, 17, 64, 65, 129])
@pytest.mark.parametrize("causal", [True, False])
def test_bwd_matches_sdpa_autograd(S, causal):
    q, k, v, do = (_rand((1, 2, S, 64), 31 * S + i) for i in range(4))
    o, lse = orc.attention_dense_fwd(q, k, v, causal=causal)
    dq, dk, dv, delta = orc.attention_bwd(q, k, v, o, lse, do, causal=causal)
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    out = _sdpa_math(tq, tk, tv, causal)
    out.backward(torch.from_numpy(do))
    assert orc.max_abs(dq, tq.grad.numpy()) < 1e-11
    assert orc.max_abs(dk, tk.grad.numpy()) < 1e-11
    assert orc.max_abs(dv, tv.grad.numpy()) < 1e-11
    assert orc.max_abs(delta, (o * do).sum(-1)) < 1e-12


def test_bwd_with_scale_matches_autograd():
    S = 77
    q, k, v, do = (_rand((1, 2, S, 64), 500 + i) for i in range(4))
    for scale in (0.3, -0.2):
        o, lse = orc.attention_dense_fwd(q, k, v, scale=scale)
        dq, dk, dv, _ = orc.attention_bwd(q, k, v, o, lse, do, scale=scale)
        tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
        out = _sdpa_math(tq, tk, tv, True, scale=scale)
        assert orc.max_abs(o, out.detach().numpy()) < 1e-12
        out.backward(torch.from_numpy(do))
        for mine, ref in ((dq, tq), (dk, tk), (dv, tv)):
            assert orc.max_abs(mine, ref.grad.numpy()) < 1e-11


def test_bwd_dropout_matches_explicit_mask_autograd():
    """p > 0: autograd of softmax(S) * keep/(1-p) @ V with the same keep mask."""
    S, p, seed = 96, 0.2, 777
    q, k, v, do = (_rand((1, 2, S, 64), 40 + i) for i in range(4))
    keep = orc.keep_mask(seed, 1, 2, S, p)
    o, lse = orc.attention_dense_fwd(q, k, v, keep=keep, p=p)
    dq, dk, dv, _ = orc.attention_bwd(q, k, v, o, lse, do, keep=keep, p=p)
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    s = torch.einsum("bhid,bhjd->bhij", tq, tk) * 0.125
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    out = torch.softmax(s, dim=-1) * torch.from_numpy(keep.astype(np.float64)) / (1 - p) @ tv
    assert orc.max_abs(o, out.detach().numpy()) < 1e-12
    out.backward(torch.from_numpy(do))
    for mine, ref in ((dq, tq), (dk, tk), (dv, tv)):
        assert orc.max_abs(mine, ref.grad.numpy()) < 1e-11


def _invariants_hold(bwd, q, k, v, do):
    """Rows of dS sum to 0 => dQ is unchanged when every key is shifted by
    the same vector; rows of P sum to 1 => sum_j dV_j = sum_i dO_i."""
    o, lse = orc.attention_dense_fwd(q, k, v)
    dq, dk, dv, _ = bwd(q, k, v, o, lse, do)
    shift = _rand((1, 1, 1, 64), 4242)
    k2 = k + shift
    o2, lse2 = orc.attention_dense_fwd(q, k2, v)
    dq2, _, _, _ = bwd(q, k2, v, o2, lse2, do)
    ok_shift = orc.max_abs(dq, dq2) < 1e-10
    ok_sum = orc.max_abs(dv.sum(axis=2), do.sum(axis=2)) < 1e-10
    return ok_shift and ok_sum


def test_bwd_invariants_and_planted_mistakes():
    S = 90
    q, k, v, do = (_rand((1, 2, S, 64), 60 + i) for i in range(4))
    assert _invariants_hold(orc.attention_bwd, q, k, v, do)

    def no_delta(q, k, v, o, lse, do):  # planted mistake: dS = P*dP (delta dropped)
        return orc.attention_bwd(q, k, v, np.zeros_like(o), lse, do)

    assert not _invariants_hold(no_delta, q, k, v, do)

    def wrong_lse(q, k, v, o, lse, do):  # planted mistake: P from lse off by one row
        return orc.attention_bwd(q, k, v, o, np.roll(lse, 1, axis=-1), do)

    assert not _invariants_hold(wrong_lse, q, k, v, do)


# --- dropout hash: each part against the published function it comes from ----------
_M = 0xFFFFFFFF


def _lowbias32_inverse(x):
    """Wellons' published inverse of lowbias32 (hash-prospector), uint64 arrays holding u32."""
    x = x ^ (x >> 16)
    x = (x * 0x43021123) & _M
    x = x ^ (x >> 15) ^ (x >> 30)
    x = (x * 0x1D69E2A5) & _M
    return x ^ (x >> 16)


def _round_trips(**planted):
    x = np.random.default_rng(11).integers(0, 2 ** 32, size=1_000_000, dtype=np.uint64)
    return np.array_equal(_lowbias32_inverse(orc.hash_u32(x, **planted)), x)


def test_dropout_finaliser_is_published_lowbias32():
    """The oracle's finaliser inverts through the published inverse on 10^6 random words."""
    assert _round_trips()


@pytest.mark.parametrize("which,bit", [(0, 0), (0, 13), (0, 30), (1, 1), (1, 22), (1, 31)])
def test_dropout_finaliser_planted_multiplier_bit(which, bit):
    mul = list(orc.LOWBIAS32_MUL)
    mul[which] ^= 1 << bit
    assert not _round_trips(mul=tuple(mul))


@pytest.mark.parametrize("which,delta", [(0, 1), (1, -1), (1, 1), (2, -1)])
def test_dropout_finaliser_planted_shift(which, delta):
    shift = list(orc.LOWBIAS32_SHIFT)
    shift[which] += delta
    assert not _round_trips(shift=tuple(shift))


def _rotl(x, r):
    return ((x << r) | (x >> (32 - r))) & _M


def _xxh32(data, seed, p1, p4):
    """XXH32 (Collet's published algorithm) with PRIME32_1 = p1 and PRIME32_4 = p4."""
    p2, p3, p5 = 0x85EBCA77, 0xC2B2AE3D, 0x165667B1
    n, i = len(data), 0
    word = lambda j: int.from_bytes(data[j:j + 4], "little")
    if n >= 16:
        v = [(seed + p1 + p2) & _M, (seed + p2) & _M, seed, (seed - p1) & _M]
        while i + 16 <= n:
            for lane in range(4):
                v[lane] = (_rotl((v[lane] + word(i + 4 * lane) * p2) & _M, 13) * p1) & _M
            i += 16
        h = (_rotl(v[0], 1) + _rotl(v[1], 7) + _rotl(v[2], 12) + _rotl(v[3], 18)) & _M
    else:
        h = (seed + p5) & _M
    h = (h + n) & _M
    while i + 4 <= n:
        h = (_rotl((h + word(i) * p3) & _M, 17) * p4) & _M
        i += 4
    while i < n:
        h = (_rotl((h + data[i] * p5) & _M, 11) * p1) & _M
        i += 1
    h ^= h >> 15
    h = (h * p2) & _M
    h ^= h >> 13
    h = (h * p3) & _M
    return h ^ (h >> 16)


def _murmur3_x86_32_u32(key, seed, f1, f2):
    """MurmurHash3_x86_32 (Appleby's published algorithm) of a 4-byte key with the
    fmix32 multipliers f1, f2."""
    k = (key * 0xCC9E2D51) & _M
    k = (_rotl(k, 15) * 0x1B873593) & _M
    h = _rotl(seed ^ k, 13)
    h = (h * 5 + 0xE6546B64) & _M
    h ^= 4
    h ^= h >> 16
    h = (h * f1) & _M
    h ^= h >> 13
    h = (h * f2) & _M
    return h ^ (h >> 16)


def _xxh32_matches(p1, p4):
    import xxhash
    rng = np.random.default_rng(12)
    for n in list(range(0, 41)) + [64, 100]:
        data = rng.integers(0, 256, size=n, dtype=np.uint8).tobytes()
        seed = int(rng.integers(0, 2 ** 32))
        if _xxh32(data, seed, p1, p4) != xxhash.xxh32_intdigest(data, seed):
            return False
    return True


def _murmur3_matches(f1, f2):
    from sklearn.utils import murmurhash3_32
    rng = np.random.default_rng(13)
    for _ in range(200):
        key, seed = int(rng.integers(-2 ** 31, 2 ** 31)), int(rng.integers(0, 2 ** 31))
        want = murmurhash3_32(key, seed=seed, positive=True)
        if _murmur3_x86_32_u32(key & _M, seed, f1, f2) != want:
            return False
    return True


def test_dropout_mixing_multipliers_are_published_constants():
    """The seed and bh multipliers are xxHash32's PRIME32_1 and PRIME32_4 (checked against
    the xxhash library), the row and col multipliers MurmurHash3's fmix32 pair (checked
    against scikit-learn's MurmurHash3_x86_32)."""
    assert _xxh32_matches(orc.DROP_SEED_MUL, orc.DROP_BH_MUL)
    assert _murmur3_matches(orc.DROP_ROW_MUL, orc.DROP_COL_MUL)
    # odd multipliers: each term is a bijection of its index modulo 2^32
    for m in (orc.DROP_SEED_MUL, orc.DROP_ROW_MUL, orc.DROP_COL_MUL, orc.DROP_BH_MUL):
        assert m & 1


@pytest.mark.parametrize("which", range(4))
@pytest.mark.parametrize("bit", [0, 7, 19, 31])
def test_dropout_mixing_planted_bit(which, bit):
    muls = [orc.DROP_SEED_MUL, orc.DROP_ROW_MUL, orc.DROP_COL_MUL, orc.DROP_BH_MUL]
    muls[which] ^= 1 << bit
    ok = _xxh32_matches(muls[0], muls[3]) and _murmur3_matches(muls[1], muls[2])
    assert not ok
    # and the oracle's hash built on the altered constant changes
    rng = np.random.default_rng(14)
    seed, row, col, bh = (rng.integers(0, 5000, size=64) for _ in range(4))
    assert not np.array_equal(orc.dropout_hash(seed, row, col, bh, muls=tuple(muls)),
                              orc.dropout_hash(seed, row, col, bh))


def test_dropout_keep_uses_the_fp32_threshold_compare():
    """keep == ((hash >> 8) * 2^-24 >= p in fp32), element for element."""
    rng = np.random.default_rng(5)
    seed = 0xC0FFEE
    row, col = rng.integers(0, 70000, size=(2, 4096))
    bh = rng.integers(0, 96, size=4096)
    h = orc.dropout_hash(seed, row, col, bh)
    for p in (0.0, 0.1, 0.5, 0.9, 1 / 3):
        u = (h >> np.uint64(8)).astype(np.float32) * np.float32(2.0 ** -24)
        assert np.array_equal(orc.dropout_keep(seed, row, col, bh, p), u >= np.float32(p))


def test_dropout_statistics():
    S, p = 512, 0.1
    keep = orc.keep_mask(123, 1, 4, S, p)
    n = keep.size
    rate = keep.mean()
    assert abs(rate - (1 - p)) < 4 * math.sqrt(p * (1 - p) / n)
    assert orc.keep_mask(0, 1, 1, 64, 0.0).all()
    assert (keep[0, 0] != keep[0, 1]).mean() > 0.1            # heads differ
    assert (keep != orc.keep_mask(124, 1, 4, S, p)).mean() > 0.1  # seeds differ
    assert (keep[0, 0] != keep[0, 0].T).mean() > 0.1           # row/col not symmetric


def _seed_golden():
    with open(os.path.join(os.path.dirname(__file__), "golden", "seed_golden.json")) as f:
        return json.load(f)["cases"]


def test_seed_formula_against_reference_vectors():
    """orc.next_seed against the seeds the reference's own _next_seed returned
    (tests/golden/make_seed_golden.py imported flash_attn_v100_cuda.py:28-33):
    14 initial seeds, including 64-bit ones, five counter values each."""
    cases = _seed_golden()
    assert len(cases) >= 10 and any(c["initial_seed"] >= 2 ** 32 for c in cases)
    for c in cases:
        assert [orc.next_seed(c["initial_seed"], i) for i in range(1, len(c["seeds"]) + 1)] == c["seeds"]


def test_seed_vectors_catch_planted_mistakes():
    """The vectors fail a seed formula with a mistyped multiplier, the counter
    starting at 0, the counter xor-ed instead of added, or a 31-bit mask."""
    cases = _seed_golden()

    def agrees(f):
        return all([f(c["initial_seed"], i) for i in range(1, 6)] == c["seeds"] for c in cases)

    assert agrees(orc.next_seed)
    assert not agrees(lambda s, i: (s * 2654435769 + i) & 0xFFFFFFFF)
    assert not agrees(lambda s, i: (s * 2654435761 + i - 1) & 0xFFFFFFFF)
    assert not agrees(lambda s, i: ((s * 2654435761) ^ i) & 0xFFFFFFFF)
    assert not agrees(lambda s, i: (s * 2654435761 + i) & 0x7FFFFFFF)


def _rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def test_rope_fwd_bitwise_vs_torch_eager():
    S = 300
    cos, sin = orc.rope_tables(S)
    tc, ts = torch.from_numpy(cos), torch.from_numpy(sin)
    x = torch.from_numpy(_rand((2, 3, S, 64), 8)).half()
    ref = (x * tc + _rotate_half(x) * ts).half()
    mine = orc.rope_fwd(x.numpy(), cos, sin)
    assert np.array_equal(mine.view(np.uint16), ref.numpy().view(np.uint16))


def test_rope_bwd_bitwise_vs_torch_autograd():
    S = 300
    cos, sin = orc.rope_tables(S)
    tc, ts = torch.from_numpy(cos), torch.from_numpy(sin)
    x = torch.from_numpy(_rand((2, 3, S, 64), 9)).float().requires_grad_(True)
    g = torch.from_numpy(_rand((2, 3, S, 64), 10)).half()
    out = x * tc + _rotate_half(x) * ts
    out.backward(g.float())
    ref = x.grad.half()
    mine = orc.rope_bwd(g.numpy(), cos, sin)
    assert np.array_equal(mine.view(np.uint16), ref.numpy().view(np.uint16))


def test_rope_tables_match_train_py_construction():
    """inv_freq over d_model 768 truncated to 64 columns: cos[:, d] != cos[:, d+32]."""
    cos, sin = orc.rope_tables(64)
    assert cos.shape == (64, 64)
    assert not np.allclose(cos[:, :32], cos[:, 32:])
    t = 5
    assert abs(cos[t, 1] - math.cos(t * 10000 ** (-2 / 768))) < 1e-6


def test_oracle_reproduces_golden_fixtures():
    """The committed fixtures (SDPA-MATH fp64 for p=0, oracle for p>0) agree
    with the oracle on the fp16 inputs they hold."""
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "fa2_golden.npz"))
    names = sorted({k.split("/")[0] for k in z.files if not k.startswith("mask")})
    assert len(names) >= 5
    for name in names:
        B, H, S, causal, scale, p, seed = z[f"{name}/meta"]
        B, H, S, seed = int(B), int(H), int(S), int(seed)
        q, k, v, do = (z[f"{name}/{t}"].astype(np.float64) for t in ("q", "k", "v", "do"))
        keep = orc.keep_mask(seed, B, H, S, p) if p > 0 else None
        if keep is not None:
            assert np.array_equal(np.packbits(keep.reshape(-1)), z[f"{name}/keepbits"])
        o, lse = orc.attention_tiled_fwd(q, k, v, causal=bool(causal), scale=scale, keep=keep, p=p)
        dq, dk, dv, _ = orc.attention_bwd(q, k, v, o, lse, do, causal=bool(causal), scale=scale, keep=keep, p=p)
        for mine, key in ((o, "o"), (lse, "lse"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
            assert orc.max_abs(mine, z[f"{name}/{key}"]) < 2e-5, (name, key)
    for key in (k for k in z.files if k.startswith("mask/")):
        _, seed, bh = key.split("/")
        rows, cols = np.arange(64).reshape(64, 1), np.arange(64).reshape(1, 64)
        assert np.array_equal(np.packbits(orc.dropout_keep(int(seed), rows, cols, int(bh), 0.1).reshape(-1)), z[key])


# ---------------------------------------------------------------------------
# Non-square forward (fa2_fwd_kv_f16's contract: key j visible to query i iff
# j <= i + causal_offset)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("Sq,Sk,coff", [(1, 70, 69), (5, 70, 65), (37, 130, 93), (64, 64, 0),
                                        (20, 150, 0), (90, 40, 0), (60, 25, -35), (33, 100, 10)])
def test_kv_fwd_matches_sdpa_math_with_explicit_mask(Sq, Sk, coff):
    q = _rand((1, 2, Sq, 64), 3 * Sq + Sk)
    k, v = (_rand((1, 2, Sk, 64), 5 * Sk + i) for i in range(2))
    o, lse = orc.attention_dense_fwd(q, k, v, causal=True, causal_offset=coff)
    vis = torch.arange(Sk)[None, :] <= torch.arange(Sq)[:, None] + coff
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    with sdpa_kernel(SDPBackend.MATH):
        ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=vis).numpy()
    s = torch.einsum("bhid,bhjd->bhij", tq, tk) * 0.125
    ref_lse = torch.logsumexp(s.masked_fill(~vis, float("-inf")), dim=-1).numpy()
    seen = vis.any(dim=1).numpy()          # rows that see no key: SDPA gives NaN, the contract 0 / -inf
    assert orc.max_abs(o[..., seen, :], ref[..., seen, :]) < 1e-12
    assert orc.max_abs(lse[..., seen], ref_lse[..., seen]) < 1e-12
    assert np.all(o[..., ~seen, :] == 0.0) and np.all(lse[..., ~seen] == -np.inf)


@pytest.mark.parametrize("Sq,Sk", [(20, 150), (90, 40), (1, 33)])
def test_kv_fwd_offset_zero_is_sdpa_is_causal(Sq, Sk):
    """torch SDPA's is_causal on non-square inputs aligns the mask top-left: offset 0."""
    q = _rand((1, 1, Sq, 64), Sq)
    k, v = (_rand((1, 1, Sk, 64), Sk + i) for i in range(2))
    o, _ = orc.attention_dense_fwd(q, k, v, causal=True, causal_offset=0)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    assert orc.max_abs(o, _sdpa_math(tq, tk, tv, True).numpy()) < 1e-12


@pytest.mark.parametrize("Sq,Sk", [(1, 70), (16, 200), (64, 64), (100, 129)])
def test_kv_fwd_bottom_right_chunk_is_tail_of_square(Sq, Sk):
    """A chunk of the last Sq queries against all Sk keys with offset Sk - Sq gives the last Sq rows
    of the square causal attention (what a KV cache must reproduce)."""
    qf, k, v = (_rand((1, 2, Sk, 64), 17 * Sk + i) for i in range(3))
    of, lf = orc.attention_dense_fwd(qf, k, v, causal=True)
    oc, lc = orc.attention_dense_fwd(qf[..., Sk - Sq:, :], k, v, causal=True, causal_offset=Sk - Sq)
    assert orc.max_abs(oc, of[..., Sk - Sq:, :]) < 1e-12
    assert orc.max_abs(lc, lf[..., Sk - Sq:]) < 1e-12


def test_kv_fwd_decode_closed_form():
    """One query against every key: softmax(q K^T * scale) V (scipy's softmax, a library routine)."""
    from scipy.special import logsumexp, softmax
    q = _rand((2, 3, 1, 64), 1)
    k, v = (_rand((2, 3, 257, 64), 2 + i) for i in range(2))
    o, lse = orc.attention_dense_fwd(q, k, v, causal=False, scale=0.2)
    s = np.einsum("bhid,bhjd->bhij", q, k) * 0.2
    assert orc.max_abs(o, np.einsum("bhij,bhjd->bhid", softmax(s, axis=-1), v)) < 1e-12
    assert orc.max_abs(lse, logsumexp(s, axis=-1)) < 1e-12


def test_reference_hash_recipe_takes_exactly_the_hash_lines():
    """oracle/build_ref.py compiles the reference's hash_u32 and dropout_keep
    (fa_common.cuh:21-38) and nothing else of the header; when the reference
    tree is present the extraction is checked here, and when the checker
    library is present it must export both harness entry points."""
    import ctypes
    import importlib.util
    spec = importlib.util.spec_from_file_location("fa2_build_ref", os.path.join(orc.__file__.rsplit("/", 1)[0], "build_ref.py"))
    br = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(br)
    if br.available():
        with open(br.HEADER) as f:
            first, block = br.extract_hash_lines(f.read())
        text = "\n".join(block)
        assert (first, first + len(block) - 1) == (21, 38)
        assert "hash_u32" in text and "dropout_keep" in text and "#include" not in text
    if os.path.exists(br.LIB):
        lib = ctypes.CDLL(br.LIB)
        assert hasattr(lib, "fa2ref_dropout_keep") and hasattr(lib, "fa2ref_hash_u32")
