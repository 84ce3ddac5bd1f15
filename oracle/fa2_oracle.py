"""CPU oracle for the causal FlashAttention-2 hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker.  The product path
(``universal-lm-trainer_amd/``) never imports it and has no CPU fallback.

NumPy restatement (float64 unless noted) of the reference's algorithm
(reference @ None):
  * forward           csrc/flash_attn_v100/flash_attn_v100.cu:109-308
  * backward formulas csrc/flash_attn_v100/flash_attn_v100_bwd.cu:10-25, 42-61, 149-191, 373-418
  * dropout hash      csrc/flash_attn_v100/fa_common.cuh:21-38
  * fused RoPE        csrc/flash_attn_v100/fast_ops.cu:31-68 (fp32, no FMA, one fp16 rounding)
  * RoPE tables       train.py:1877-1918

How each function is pinned (tests/test_oracle.py):
  attention_dense_fwd  torch SDPA MATH backend (fp64, a library routine) on the same
                       inputs; closed forms (row 0 = V0; Q = 0 gives the cumulative
                       mean and LSE_i = ln(i+1)); brute force on tiny shapes.
                       Non-square (causal_offset): SDPA MATH with the explicit
                       boolean mask and with is_causal (top-left, offset 0); a
                       bottom-right chunk equals the last rows of the square
                       causal result; decode (one query, all keys visible) equals
                       softmax(q K^T) V from scipy.
  attention_tiled_fwd  the dense oracle (fp64, ~1e-12) including tails (S % 64 != 0)
                       and the -inf / l = 0 guards.
  attention_bwd        torch autograd of SDPA MATH (fp64); invariants (rows of dS sum
                       to 0 so dQ is invariant to shifting all keys; sum of dV rows =
                       sum of dO rows at p = 0); torch autograd of an explicit-mask
                       dropout attention for p > 0.
  dropout_keep         the finaliser against Wellons' published inverse of lowbias32
                       (round trip on 10^6 words); the four input multipliers
                       against the published algorithms they come from (xxHash32
                       via the ``xxhash`` library, MurmurHash3_x86_32 via
                       scikit-learn); the fp32 threshold compare against the
                       integer form the kernels use, over all 2^24 values; planted
                       one-bit mistakes in every constant and shift fail those
                       checks.  Which index takes which multiplier (and the +1
                       offsets) is restated from the source text; the reference
                       holds no golden masks to pin it further.
  rope_fwd / rope_bwd  torch eager fp32 expression (train.py:1904-1918) and its fp32
                       autograd, then .half(): bitwise.
"""

import numpy as np

LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453

# ---------------------------------------------------------------------------
# dropout hash (fa_common.cuh:21-38)
# ---------------------------------------------------------------------------
_M32 = np.uint64(0xFFFFFFFF)

# Finaliser (fa_common.cuh:21-26): Wellons' published "lowbias32"
# (hash-prospector), x ^= x >> 16; x *= M1; x ^= x >> 15; x *= M2; x ^= x >> 16.
LOWBIAS32_MUL = (0x7FEB352D, 0x846CA68B)
LOWBIAS32_SHIFT = (16, 15, 16)
# Input mixing (fa_common.cuh:32-35): seed, row + 1, col + 1 and bh + 1 times
# these multipliers, xor-ed.  They are published constants: xxHash32's
# PRIME32_1 (seed) and PRIME32_4 (bh), MurmurHash3's fmix32 multipliers (row,
# col); tests/test_oracle.py checks each against those algorithms.
DROP_SEED_MUL = 0x9E3779B1
DROP_ROW_MUL = 0x85EBCA6B
DROP_COL_MUL = 0xC2B2AE35
DROP_BH_MUL = 0x27D4EB2F


def _u32(x):
    return (np.asarray(x, dtype=np.uint64) & _M32)


def hash_u32(x, mul=LOWBIAS32_MUL, shift=LOWBIAS32_SHIFT):
    """lowbias32 finaliser (fa_common.cuh:21-26), vectorised over uint64 holding u32.

    ``mul``/``shift`` default to the reference's; tests pass altered ones to
    plant a mistake."""
    x = _u32(x)
    x = x ^ (x >> np.uint64(shift[0]))
    x = (x * np.uint64(mul[0])) & _M32
    x = x ^ (x >> np.uint64(shift[1]))
    x = (x * np.uint64(mul[1])) & _M32
    x = x ^ (x >> np.uint64(shift[2]))
    return x


def dropout_hash(seed, row, col, bh, muls=None):
    """The 32-bit hash of (seed, query row, key col, b*H+h) (fa_common.cuh:30-36).

    ``muls`` = (seed, row, col, bh) multipliers, the reference's by default."""
    ms, mr, mc, mb = muls or (DROP_SEED_MUL, DROP_ROW_MUL, DROP_COL_MUL, DROP_BH_MUL)
    h = (_u32(seed) * np.uint64(ms)) & _M32
    h = h ^ ((_u32(np.asarray(row, np.int64) + 1) * np.uint64(mr)) & _M32)
    h = h ^ ((_u32(np.asarray(col, np.int64) + 1) * np.uint64(mc)) & _M32)
    h = h ^ ((_u32(np.asarray(bh, np.int64) + 1) * np.uint64(mb)) & _M32)
    return hash_u32(h)


def dropout_keep(seed, row, col, bh, p):
    """keep mask of (seed, query row, key col, b*H+h) (fa_common.cuh:30-38).

    ``row``/``col``/``bh`` broadcast.  keep iff (h >> 8) * 2^-24 >= p with the
    compare done in fp32 as the reference does."""
    h = dropout_hash(seed, row, col, bh)
    u = (h >> np.uint64(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    return u >= np.float32(p)


def keep_mask(seed, B, H, S, p):
    """Full [B,H,S,S] keep mask (query rows, key cols) for bh = b*H + h."""
    bh = np.arange(B * H).reshape(B, H, 1, 1)
    row = np.arange(S).reshape(1, 1, S, 1)
    col = np.arange(S).reshape(1, 1, 1, S)
    return dropout_keep(seed, row, col, bh, p)


def next_seed(initial_seed, counter):
    """(initial_seed * 2654435761 + counter) & 0xFFFFFFFF (flash_attn_v100_cuda.py:32-33)."""
    return (int(initial_seed) * 2654435761 + int(counter)) & 0xFFFFFFFF


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------
def _visible(S, causal, Sk=None, causal_offset=0):
    """[S, Sk] visibility: key j visible to query i iff j <= i + causal_offset (causal)."""
    Sk = S if Sk is None else Sk
    if not causal:
        return np.ones((S, Sk), dtype=bool)
    return np.arange(Sk)[None, :] <= np.arange(S)[:, None] + causal_offset


def attention_dense_fwd(q, k, v, causal=True, scale=None, keep=None, p=0.0, causal_offset=0):
    """Dense fp64 attention.  q: [B,H,S,D], k, v: [B,H,Sk,D] (Sk = S in the
    reference's square case).  Returns (O, LSE).

    LSE is the natural-log logsumexp of the scaled visible scores (-inf if a
    row sees nothing, flash_attn_v100.cu:283-287); P uses the un-dropped
    softmax and dropout multiplies it by keep/(1-p) (flash_attn_v100.cu:208-231);
    a row with l = 0 gives O = 0 (:280).  causal_offset generalises the mask to
    non-square inputs (key j visible to query i iff j <= i + causal_offset),
    the fa2_fwd_kv_f16 contract; the reference itself is square-only."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    S, D = q.shape[-2], q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    vis = _visible(S, causal, k.shape[-2], causal_offset)
    s = np.where(vis, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    e = np.where(vis, np.exp(s - m_safe), 0.0)
    l = e.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        lse = np.where(l > 0, m_safe + np.log(np.where(l > 0, l, 1.0)), -np.inf)[..., 0]
    P = np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0)
    if keep is not None and p > 0:
        P = P * keep / (1.0 - p)
    o = np.einsum("bhij,bhjd->bhid", P, v)
    return o, lse


def attention_tiled_fwd(q, k, v, causal=True, scale=None, keep=None, p=0.0, tile=64,
                        round_p_fp16=False):
    """FA-2 online softmax in the reference's step order (flash_attn_v100.cu:109-308).

    Works in the log2 domain: x = s * scale*log2e; per key tile: mask to -inf,
    m_new = max(m, rowmax x); alpha = exp2(m - m_new) (0 if m_new = -inf);
    P = exp2(x - m_new); l = l*alpha + rowsum(P) (un-dropped); optional
    dropout on P; acc = acc*alpha + P V.  Epilogue O = acc / l (0 if l = 0),
    LSE = (m + log2 l) * ln2.  ``round_p_fp16`` rounds P to fp16 before PV as
    the GPU kernels do."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    B, H, S, D = q.shape
    if scale is None:
        scale = D ** -0.5
    scale2 = scale * LOG2E
    o = np.zeros((B, H, S, D))
    lse = np.zeros((B, H, S))
    rows = np.arange(S)
    for b in range(B):
        for h in range(H):
            for m0 in range(0, S, tile):
                r = rows[m0:m0 + tile]
                qt = q[b, h, r]
                acc = np.zeros((len(r), D))
                mrow = np.full(len(r), -np.inf)
                lrow = np.zeros(len(r))
                hi = min(S, m0 + tile) if causal else S
                for n0 in range(0, hi, tile):
                    cidx = np.arange(n0, min(n0 + tile, S))
                    x = (qt @ k[b, h, cidx].T) * scale2
                    if causal:
                        x = np.where(cidx[None, :] > r[:, None], -np.inf, x)
                    mnew = np.maximum(mrow, x.max(axis=1))
                    fin = np.isfinite(mnew)
                    with np.errstate(invalid="ignore"):
                        alpha = np.where(fin, np.exp2(np.where(fin, mrow - np.where(fin, mnew, 0), 0)), 0.0)
                    sub = np.where(fin, mnew, 0.0)
                    P = np.exp2(x - sub[:, None])
                    lrow = lrow * alpha + P.sum(axis=1)
                    if keep is not None and p > 0:
                        P = P * keep[b, h][np.ix_(r, cidx)] / (1.0 - p)
                    if round_p_fp16:
                        P = P.astype(np.float16).astype(np.float64)
                    acc = acc * alpha[:, None] + P @ v[b, h, cidx]
                    mrow = mnew
                inv = np.where(lrow > 0, 1.0 / np.where(lrow > 0, lrow, 1.0), 0.0)
                o[b, h, r] = acc * inv[:, None]
                with np.errstate(divide="ignore"):
                    lse[b, h, r] = np.where(np.isfinite(mrow),
                                            (mrow + np.log2(np.where(lrow > 0, lrow, 1.0))) * LN2,
                                            -np.inf)
    return o, lse


# ---------------------------------------------------------------------------
# backward (flash_attn_v100_bwd.cu:10-25)
# ---------------------------------------------------------------------------
def attention_bwd(q, k, v, o, lse, do, causal=True, scale=None, keep=None, p=0.0):
    """Returns (dq, dk, dv, delta) in fp64.

    delta = rowsum(O * dO) (bwd.cu:42-61); P = exp(scale*QK^T - lse) on visible
    entries; P_d = keep * P / (1-p); dP = dO V^T; dS = P_d * dP - P * delta;
    dV = P_d^T dO; dQ = scale * dS K; dK = scale * dS^T Q."""
    q, k, v, o, do = (np.asarray(t, np.float64) for t in (q, k, v, o, do))
    lse = np.asarray(lse, np.float64)
    S, D = q.shape[-2], q.shape[-1]
    if scale is None:
        scale = D ** -0.5
    delta = (o * do).sum(axis=-1)
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    vis = _visible(S, causal)
    P = np.where(vis, np.exp(np.where(vis, s, 0.0) - lse[..., None]), 0.0)
    Pd = P * keep / (1.0 - p) if (keep is not None and p > 0) else P
    dP = np.einsum("bhid,bhjd->bhij", do, v)
    dS = Pd * dP - P * delta[..., None]
    dv = np.einsum("bhij,bhid->bhjd", Pd, do)
    dq = scale * np.einsum("bhij,bhjd->bhid", dS, k)
    dk = scale * np.einsum("bhij,bhid->bhjd", dS, q)
    return dq, dk, dv, delta


# ---------------------------------------------------------------------------
# RoPE (train.py:1877-1918, fast_ops.cu:31-68)
# ---------------------------------------------------------------------------
def rope_tables(seq_len, d_model=768, head_dim=64, base=10000.0):
    """cos/sin [S, head_dim] fp32 as train.py builds them: inv_freq over
    d_model, emb = cat(freqs, freqs), sliced to head_dim (train.py:1882-1906)."""
    inv_freq = (1.0 / (base ** (np.arange(0, d_model, 2, dtype=np.float32) / np.float32(d_model)))).astype(np.float32)
    t = np.arange(seq_len, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb)[:, :head_dim].astype(np.float32), np.sin(emb)[:, :head_dim].astype(np.float32)


def rope_fwd(x, cos, sin):
    """out = x*cos + rotate_half(x)*sin in fp32 (separate rounding), then fp16."""
    x = np.asarray(x).astype(np.float32)
    rot = np.concatenate([-x[..., 32:], x[..., :32]], axis=-1)
    out = (x * cos.astype(np.float32)).astype(np.float32) + (rot * sin.astype(np.float32)).astype(np.float32)
    return out.astype(np.float32).astype(np.float16)


def rope_bwd(g, cos, sin):
    """gx[d] = g[d]*cos[d] + t[d], t = (+g[d+32]*sin[d+32] | -g[d-32]*sin[d-32]), fp32 then fp16."""
    g = np.asarray(g).astype(np.float32)
    gs = (g * sin.astype(np.float32)).astype(np.float32)
    t = np.concatenate([gs[..., 32:], -gs[..., :32]], axis=-1)
    out = (g * cos.astype(np.float32)).astype(np.float32) + t
    return out.astype(np.float32).astype(np.float16)


# ---------------------------------------------------------------------------
# comparison metrics used by the parity tests
# ---------------------------------------------------------------------------
def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b.ravel())
    return float(np.linalg.norm((a - b).ravel()) / den) if den > 0 else float(np.linalg.norm(a.ravel()))
