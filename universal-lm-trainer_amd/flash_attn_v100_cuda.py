"""flash_attn_v100_cuda -- drop-in replacement of the reference's loader/op layer,
backed by hand-written gfx950 (MI355X) HIP kernels.

Same module name and public API as the reference (reference @ None:
flash_attn_v100_cuda.py:1-166), so ``train.py`` picks it up unchanged with
``sys.path`` pointing at this directory:

    is_available() -> bool            build_error() -> Exception | None
    can_use(q, k, v) -> bool          flash_attn_v100(q, k, v, dropout_p=0.0,
                                                      causal=True, softmax_scale=None)
    rope_can_use(q, k, cos, sin)      rope(q, k, cos2d, sin2d) -> (q_out, k_out)

Differences of mechanism, not of contract:
  * ``_build()`` loads the prebuilt in-tree extension ``lib/_fa2_torch*.so``
    (built by ``build.py``; no JIT compile at import).  A missing or broken
    build is recorded as ``build_error()`` and ``is_available()`` is False,
    exactly as the reference reports a failed JIT build.  Calling
    ``flash_attn_v100`` without the extension raises ``RuntimeError``; there is
    no silent fallback inside the op -- the SDPA fallback belongs to the caller
    (``train.py:1955-1961``), and ``sdpa()`` below reproduces that decision for
    callers that want it in one place.
  * Kernels accept 16-byte alignment; ``can_use`` keeps the reference's
    stricter 32-byte predicate so the same tensors are routed the same way.

Additions used by inference callers (``inf.py:128-133``,
``hf_template/modeling_universal_lm.py:149-153``):
  * ``sdpa(...)`` has the signature of
    ``torch.nn.functional.scaled_dot_product_attention``.  With no mask it
    sends the causal, ``can_use`` case to ``flash_attn_v100`` (training,
    differentiable) and, when no gradient is needed and there is no dropout,
    any other fp16 head-64 shape -- non-causal, or ``S_q != S_k`` such as
    decode against a KV cache -- to the forward kernel with SDPA's semantics
    (``is_causal`` aligned top-left).  Everything else calls SDPA unchanged.
  * ``flash_attn_kvcache(q, k, v, causal=True)``: forward-only attention of a
    chunk of ``S_q`` new queries against ``S_k`` cached keys with the causal
    mask aligned bottom-right (the chunk is the last ``S_q`` positions), the
    mask the HF template builds by hand for KV-cache chunks
    (``hf_template/modeling_universal_lm.py:228-246``).
"""

import glob
import importlib.util
import itertools
import os

import torch
import torch.nn.functional as F

_THIS_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB_DIR = os.path.join(_THIS_DIR, "lib")

_EXT = None
_BUILD_ERROR = None

# The backward must reuse the forward's dropout mask.  The mask is a pure
# function of (seed, row, col, bh), so the seed (saved in ctx) is enough for
# the backward to hash it again; the keep-bit words below only spare it that
# work.
_SEED_COUNTER = itertools.count(1)

# Keep-bit words: with dropout, and only when a gradient of q, k or v will be
# computed, the forward also stores its keep bits (one bit per query/key pair
# it computes: 104 MB at B=8 H=12 S=4096 causal, 201 MB without the causal
# mask), saved with the other tensors until the backward, which then reads
# them instead of hashing again: identical gradients, less backward work.
# The words live as long as the autograd graph
# holds them, i.e. one set per attention call awaiting its backward (ten for a
# ten-layer model).  This cap applies to each call's words on their own, not to
# their total: a call whose words would exceed it hashes in the backward
# instead (seed only), and a cap of 0 turns the words off.
def _mask_cap(default=1 << 30):
    text = os.environ.get("FA_V100_DROPOUT_MASK_MAX_BYTES", "")
    try:
        return int(text) if text.strip() else default
    except ValueError:   # a malformed setting must not break the import (and train.py with it)
        return default


DROPOUT_MASK_MAX_BYTES = _mask_cap()


def dropout_mask_bytes(B, H, S, causal=False):
    """Bytes of the keep-bit words of a (B, H, S) call (fa2_dropout_mask_bytes,
    or fa2_dropout_mask_bytes_causal with the causal mask)."""
    J, R = (S + 127) // 128, (S + 255) // 256 * 256
    words = 4 * J * R - 256 * J * (J - 1) if causal else 4 * J * R
    return B * H * words * 4


def _next_seed():
    """Seed of the next dropout mask (reference flash_attn_v100_cuda.py:32-33)."""
    return (int(torch.cuda.initial_seed()) * 2654435761 + next(_SEED_COUNTER)) & 0xFFFFFFFF


def _ext_file():
    hits = sorted(glob.glob(os.path.join(_LIB_DIR, "_fa2_torch*.so")))
    return hits[0] if hits else None


def _build():
    """Load the prebuilt extension once; record the failure reason otherwise."""
    global _EXT, _BUILD_ERROR
    if _EXT is not None or _BUILD_ERROR is not None:
        return
    try:
        path = _ext_file()
        if path is None:
            raise ImportError(
                f"gfx950 attention extension not built (no _fa2_torch*.so under {_LIB_DIR}); "
                "run `python universal-lm-trainer_amd/build.py`")
        spec = importlib.util.spec_from_file_location("_fa2_torch", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _EXT = mod
    except Exception as e:  # recorded, reported through build_error()
        _BUILD_ERROR = e
        _EXT = None


def is_available():
    _build()
    return _EXT is not None


def build_error():
    _build()
    return _BUILD_ERROR


def extension():
    """The loaded extension module; raises RuntimeError if it is not built."""
    _build()
    if _EXT is None:
        raise RuntimeError(f"flash_attn_v100 (gfx950) extension unavailable: {_BUILD_ERROR}")
    return _EXT


class _FlashAttnV100Cuda(torch.autograd.Function):
    """autograd Function over fa_fwd / fa_bwd (reference flash_attn_v100_cuda.py:69-94)."""

    @staticmethod
    def forward(ctx, q, k, v, dropout_p, causal, softmax_scale):
        ext = extension()
        seed = _next_seed()
        mask = None
        if (dropout_p > 0 and any(ctx.needs_input_grad[:3])
                and dropout_mask_bytes(*q.shape[:3], causal=bool(causal)) <= DROPOUT_MASK_MAX_BYTES):
            o, lse, mask = ext.fa_fwd_mask(q, k, v, float(dropout_p), bool(causal), float(softmax_scale), int(seed))
        else:
            o, lse = ext.fa_fwd(q, k, v, float(dropout_p), bool(causal), float(softmax_scale), int(seed))
        ctx.save_for_backward(q, k, v, o, lse, mask)
        ctx.dropout_p = float(dropout_p)
        ctx.causal = bool(causal)
        ctx.softmax_scale = float(softmax_scale)
        ctx.seed = int(seed)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, mask = ctx.saved_tensors
        ext = extension()
        if not hasattr(ext, "fa_bwd"):
            raise NotImplementedError("flash_attn_v100: backward kernel missing from the extension")
        # The kernels read dO through its strides; only rows must be contiguous.
        dq, dk, dv = ext.fa_bwd(q, k, v, o, lse, do if do.stride(3) == 1 else do.contiguous(),
                                ctx.dropout_p, ctx.causal, ctx.softmax_scale, ctx.seed, 7, mask=mask)
        return dq, dk, dv, None, None, None


def _fa_ready(t):
    """fp16, (B,H,S,64), last dim contiguous, 32-byte aligned base and strides
    (reference flash_attn_v100_cuda.py:97-102)."""
    return (t.is_cuda and t.dtype == torch.float16 and t.dim() == 4
            and t.size(3) == 64 and t.stride(3) == 1
            and t.data_ptr() % 32 == 0
            and all((s * 2) % 32 == 0 for s in t.stride()[:3]))


def can_use(q, k, v):
    """Whether the tensors can go to the kernel directly (reference :105-108)."""
    return (_fa_ready(q) and _fa_ready(k) and _fa_ready(v)
            and q.shape == k.shape == v.shape)


class _RopeV100Cuda(torch.autograd.Function):
    """Fused RoPE, one kernel each way (reference flash_attn_v100_cuda.py:111-138)."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        qo, ko = extension().rope_fwd(q, k, cos, sin)
        ctx.save_for_backward(q, k, cos, sin)
        return qo, ko

    @staticmethod
    def backward(ctx, dqo, dko):
        q, k, cos, sin = ctx.saved_tensors
        q_unused, k_unused = dqo is None, dko is None
        if q_unused and k_unused:
            return None, None, None, None
        if q_unused:
            dqo = torch.zeros_like(q)
        elif dqo.stride(3) != 1:
            dqo = dqo.contiguous()
        if k_unused:
            dko = torch.zeros_like(k)
        elif dko.stride(3) != 1:
            dko = dko.contiguous()
        dq, dk = extension().rope_bwd(dqo, dko, cos, sin, q, k)
        return (None if q_unused else dq), (None if k_unused else dk), None, None


def rope_can_use(q, k, cos, sin):
    """Eligibility of the fused RoPE (reference flash_attn_v100_cuda.py:141-147)."""
    return (is_available() and _fa_ready(q) and _fa_ready(k)
            and q.shape == k.shape
            and cos.dtype == torch.float32 and sin.dtype == torch.float32
            and cos.device == q.device and sin.device == q.device
            and cos.shape == (q.size(2), 64) and sin.shape == cos.shape
            and cos.stride(1) == 1 and sin.stride(1) == 1)


def rope(q, k, cos2d, sin2d):
    """q, k: (B,H,S,64) fp16 strided views; cos2d/sin2d: (S,64) fp32 (rows may be padded)."""
    return _RopeV100Cuda.apply(q, k, cos2d, sin2d)


def flash_attn_v100(q, k, v, dropout_p: float = 0.0, causal: bool = True, softmax_scale=None):
    """Causal FlashAttention-2 on MI355X; same contract as the reference (:155-166)."""
    if not (q.is_cuda and q.dtype == torch.float16 and q.size(3) == 64):
        raise ValueError("flash_attn_v100 only supports fp16 GPU tensors with head_dim=64")
    if not _fa_ready(q) or not _fa_ready(k) or not _fa_ready(v):
        q, k, v = (t if _fa_ready(t) else t.contiguous() for t in (q, k, v))
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    return _FlashAttnV100Cuda.apply(q, k, v, float(dropout_p), bool(causal), float(softmax_scale))


def _disabled():
    return os.environ.get("FA_V100_DISABLE", "0") == "1"


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def _kv_ready(q, k, v):
    """fp16 (B,H,S_q,64) queries against (B,H,S_k,64) keys/values, kernel-aligned."""
    return (_fa_ready(q) and _fa_ready(k) and _fa_ready(v) and k.shape == v.shape
            and k.shape[:2] == q.shape[:2] and k.size(2) >= 1)


def _fwd_kv(q, k, v, causal, softmax_scale, causal_offset):
    if not (q.is_cuda and q.dtype == torch.float16 and q.dim() == 4 and q.size(3) == 64):
        raise ValueError("fp16 GPU tensors (B,H,S,64) only")
    if _needs_grad(q, k, v):
        raise RuntimeError("the key/value-length forward is inference-only (no backward)")
    q, k, v = (t if _fa_ready(t) else t.contiguous() for t in (q, k, v))
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    o, _ = extension().fa_fwd_kv(q, k, v, bool(causal), float(softmax_scale), int(causal_offset))
    return o


def flash_attn_kvcache(q, k, v, causal: bool = True, softmax_scale=None):
    """Attention of q (B,H,S_q,64) against k, v (B,H,S_k,64), forward only, for
    inference: a prefill chunk against a KV cache, or decode (S_q = 1).  With
    causal, query i sees keys j <= i + S_k - S_q (the chunk is the last S_q
    positions: the mask of hf_template/modeling_universal_lm.py:228-246); a
    query that sees no key (S_q > S_k) gets zeros.  No reference counterpart:
    the reference's kernel is square-only and these callers use SDPA."""
    return _fwd_kv(q, k, v, causal, softmax_scale, k.size(2) - q.size(2))


def sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, **kwargs):
    """Signature of ``F.scaled_dot_product_attention``.  Mask-free calls go to
    the kernels: the causal ``can_use`` case through ``flash_attn_v100`` (the
    decision of train.py:1946-1961), and, when no gradient is needed and
    dropout is 0, other fp16 head-64 shapes (non-causal, S_q != S_k) through
    the forward with SDPA's semantics.  Everything else calls SDPA unchanged."""
    eligible = attn_mask is None and not kwargs and not _disabled() and is_available() and query.dim() == 4
    if eligible and is_causal and can_use(query, key, value):
        return flash_attn_v100(query, key, value, dropout_p=dropout_p, causal=True,
                               softmax_scale=scale)
    if (eligible and dropout_p == 0.0 and query.dtype == torch.float16 and query.size(3) == 64
            and _kv_ready(query, key, value) and not _needs_grad(query, key, value)):
        # SDPA semantics: is_causal on S_q != S_k aligns the mask top-left (offset 0).
        return _fwd_kv(query, key, value, is_causal, scale, 0)
    return F.scaled_dot_product_attention(query, key, value, attn_mask=attn_mask,
                                          dropout_p=dropout_p, is_causal=is_causal,
                                          scale=scale, **kwargs)
