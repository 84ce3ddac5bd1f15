/*
 * fa2_mi355x.h -- C ABI of the MI355X (gfx950) causal FlashAttention-2 library.
 *
 * Plain C: pointers, sizes and element strides only; no torch or HIP types in
 * the signatures (streams are passed as `void*`, i.e. a hipStream_t, NULL =
 * the null stream).  Every entry point
 *   - validates its arguments and returns a status code (0 = success),
 *   - allocates nothing (outputs and workspace belong to the caller),
 *   - launches asynchronously on the given stream and never synchronises,
 *   - keeps no state between calls, so it is reentrant and may be called from
 *     any host thread (the autograd engine calls the backward from its own
 *     device thread).
 *
 * Tensor convention (the reference's): a 4-D fp16 tensor [B, H, S, D] with
 * D == 64, the last dimension contiguous, and arbitrary element strides for
 * (b, h, s).  Strides must be multiples of 8 elements and base pointers
 * 16-byte aligned (the kernels move 16-byte vectors); the reference demands
 * 32 bytes (reference @ None: flash_attn_v100_cuda.py:97-102), so every
 * tensor it accepts is accepted here.
 */
#ifndef FA2_MI355X_H
#define FA2_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA2_HEAD_DIM 64

/* Status codes. */
enum fa2_status {
    FA2_OK = 0,
    FA2_ERR_NULL_POINTER = 1,   /* a required pointer is NULL                 */
    FA2_ERR_BAD_SHAPE = 2,      /* B/H/S negative, D != 64, int32 overflow   */
    FA2_ERR_MISALIGNED = 3,     /* pointer or stride breaks 16-byte alignment */
    FA2_ERR_BAD_ARGUMENT = 4,   /* dropout_p outside [0,1), bad mode bits ... */
    FA2_ERR_WORKSPACE = 5,      /* workspace missing or too small            */
    FA2_ERR_LAUNCH = 6          /* the HIP runtime rejected a kernel launch   */
};

/* Forward: O = softmax(scale * Q K^T [+ causal mask]) V, with dropout on P,
 * and LSE[b,h,i] = natural-log logsumexp of row i of the scaled, masked
 * scores (-inf for a row with no visible key).
 * Replaces fav100::fa_fwd / fa_fwd_kernel
 *   (reference @ None: csrc/flash_attn_v100/flash_attn_v100.cu:40-364). */
typedef struct fa2_fwd_params {
    const void *q, *k, *v;          /* fp16 [B,H,S,64]                         */
    void *o;                        /* fp16 [B,H,S,64] output                  */
    float *lse;                     /* fp32 [B,H,S] output                     */
    int64_t q_stride[3], k_stride[3], v_stride[3], o_stride[3]; /* b,h,s     */
    int64_t lse_stride[2];          /* b,h (the s stride is 1)                 */
    int32_t B, H, S, D;
    float softmax_scale;            /* the reference default is D^-0.5         */
    float dropout_p;                /* 0 <= p < 1                              */
    uint32_t seed;                  /* dropout hash seed                       */
    int32_t causal;                 /* nonzero: key j visible to query i iff j <= i */
    uint32_t *dropout_mask;         /* optional keep-bit output, see below; NULL = none */
    size_t dropout_mask_bytes;      /* bytes at dropout_mask: with dropout_p > 0 at least
                                       fa2_dropout_mask_bytes_causal(B, H, S) when causal,
                                       fa2_dropout_mask_bytes(B, H, S) otherwise, else
                                       FA2_ERR_WORKSPACE (ignored when dropout_mask is NULL) */
} fa2_fwd_params;

int fa2_fwd_f16(const fa2_fwd_params *p, void *stream);

/* Dropout keep bits.  With dropout_p > 0 and dropout_mask non-NULL,
 * fa2_fwd_f16 also stores the keep bit of every (query, key) pair it computes
 * -- the same bits its dropout hash draws -- into dropout_mask
 * (fa2_dropout_mask_bytes_causal(B, H, S) bytes with the causal mask,
 * fa2_dropout_mask_bytes(B, H, S) without, 16-byte aligned; words it does not
 * compute, such as those of queries a key tile only partly reaches, are left
 * as they were).
 * fa2_bwd_f16 given the same words in its dropout_mask (with the same B, H,
 * S, causal, dropout_p and seed) reads them instead of hashing again: the
 * results are identical, the backward's hash work is gone, and the words cost
 * one bit per pair of HBM (written once, read by the dQ and dK/dV passes).
 * The fa2_fwd_kv_* entry points take no mask (dropout_mask must be NULL).
 * No counterpart in the reference, which draws its dropout with curand in
 * the forward only (reference @ None: csrc/flash_attn_v100/flash_attn_v100.cu:40-364).
 * Word layout, per (b, h), 64-key tile t (< T = 2*ceil(S/128)), half g (0, 1)
 * and query i (< R = S rounded up to 256); the word's bit
 * 31 - (16*kb + 8*hh + e) is key 64*t + 32*kb + 16*hh + 8*(e/4) + 4*g + e%4
 * (kb, hh in 0..1, e in 0..7).
 *   - Without the causal mask: word ((b*H + h)*T + t)*2*R + g*R + i.
 *   - With it, tile t keeps queries i >= r = 128*(t/2) only (earlier queries
 *     see none of its keys), in runs of n = R - r words: word
 *     (b*H + h)*W(T/2) + W(t/2) + (t%2)*2*n + g*n + (i - r), where
 *     W(j) = 4*j*R - 256*j*(j-1) counts the words of the tiles before 2*j.
 *     That is about half of the square layout's bytes. */
size_t fa2_dropout_mask_bytes(int32_t B, int32_t H, int32_t S);
/* Bytes of the keep-bit words of a causal call: B*H*W(T/2)*4 (see above). */
size_t fa2_dropout_mask_bytes_causal(int32_t B, int32_t H, int32_t S);

/* The integer form of the reference's keep test, which every kernel uses:
 * (h >> 8) * 2^-24 >= p in fp32 (exact, since h >> 8 < 2^24) holds iff
 * (h >> 8) >= fa2_dropout_threshold(p) = ceil(p * 2^24).  A host function (no
 * GPU needed), exported so that the equivalence can be checked exhaustively.
 * Replaces the compare of dropout_keep
 *   (reference @ None: csrc/flash_attn_v100/fa_common.cuh:37). */
uint32_t fa2_dropout_threshold(float dropout_p);

/* Forward over a key/value sequence of its own length, for inference callers:
 * a prefill chunk of S new queries against a KV cache of s_k rows, or decode
 * (S = 1).  Same as fa2_fwd_f16 except that k and v are [B,H,s_k,64] (q, o
 * and lse keep S rows) and, with causal set, key j is visible to query i iff
 * j <= i + causal_offset: 0 is torch SDPA's is_causal alignment (top-left),
 * s_k - S the KV-cache one (bottom-right: the chunk is the last S positions).
 * A query that sees no key gets O = 0 and LSE = -inf.  s_k = S with
 * causal_offset = 0 is fa2_fwd_f16, bit for bit, except for S = 1 without
 * dropout (decode), which takes a kernel of its own (equal to rounding).
 * No counterpart in the reference, whose kernel is square-only: its inference
 * paths call torch SDPA on exactly these shapes (reference @ None: inf.py:128-133,
 * hf_template/modeling_universal_lm.py:149-153 with the masks of :228-251). */
int fa2_fwd_kv_f16(const fa2_fwd_params *p, int32_t s_k, int32_t causal_offset, void *stream);

/* fa2_fwd_kv_f16 with the key range cut into nsplit slices of equal whole
 * 64-key tiles, run as nsplit times as many workgroups, whose partial results
 * (O accumulator, max, row sum per query) a second kernel merges -- for shapes
 * with too few query blocks to fill the GPU (decode, short chunks).  Needs
 * fa2_fwd_kv_workspace_bytes(B, H, S, nsplit) bytes of workspace, 16-byte
 * aligned; nsplit = 1 is fa2_fwd_kv_f16 and needs none.  1 <= nsplit <= 1024
 * and B*H*ceil(S/128)*nsplit < 2^31 (the grid), else FA2_ERR_BAD_SHAPE.
 * Same results as fa2_fwd_kv_f16 up to fp32 rounding of the merge.
 * No counterpart in the reference (see fa2_fwd_kv_f16). */
size_t fa2_fwd_kv_workspace_bytes(int32_t B, int32_t H, int32_t S, int32_t nsplit);
int fa2_fwd_kv_split_f16(const fa2_fwd_params *p, int32_t s_k, int32_t causal_offset, int32_t nsplit,
                         void *workspace, size_t workspace_bytes, void *stream);

/* Backward: dQ, dK, dV from Q, K, V, O, LSE and dO, recomputing P from LSE.
 * Replaces fav100::fa_bwd and its three kernels (delta, dQ, dK/dV)
 *   (reference @ None: csrc/flash_attn_v100/flash_attn_v100_bwd.cu:42-506).
 * `mode` keeps the reference's bit mask (bwd.cu:476-502), 1 = delta,
 * 2 = dQ, 4 = dK/dV, 7 = all (0..7; anything else is FA2_ERR_BAD_ARGUMENT):
 *   - 7: split pass like the reference -- a dQ kernel that also writes delta,
 *     then the dK/dV kernel (no atomics, run-to-run identical);
 *   - 2: the dQ kernel (writes delta); 1: delta only; 4: dK/dV reading the
 *     delta and scaled LSE an earlier call (mode 1 or 2) left in the
 *     workspace.
 * The workspace (fa2_bwd_workspace_bytes) holds delta[b,h,i] = sum_d O*dO and
 * LSE[b,h,i] * log2(e) in fp32 and the per-row terms -LSE*log2(e)/scale2 and
 * -delta that start the dK/dV step's accumulators (all written by the dQ or
 * delta step, read by the dK/dV step).  B*H*S must be below 2^30. */
typedef struct fa2_bwd_params {
    const void *q, *k, *v, *o, *dout;   /* fp16 [B,H,S,64]                     */
    const float *lse;                   /* fp32 [B,H,S] from the forward       */
    void *dq, *dk, *dv;                 /* fp16 [B,H,S,64] outputs             */
    int64_t q_stride[3], k_stride[3], v_stride[3], o_stride[3], do_stride[3];
    int64_t dq_stride[3], dk_stride[3], dv_stride[3];
    int64_t lse_stride[2];
    int32_t B, H, S, D;
    float softmax_scale;
    float dropout_p;
    uint32_t seed;
    int32_t causal;
    const uint32_t *dropout_mask;       /* optional: fa2_fwd_f16's keep bits (see
                                           fa2_dropout_mask_bytes), read by the dQ
                                           and dK/dV kernels instead of the hash,
                                           with the same result; NULL = hash      */
    size_t dropout_mask_bytes;          /* bytes at dropout_mask, checked like the
                                           forward's                              */
} fa2_bwd_params;

/* Workspace bytes fa2_bwd_f16 needs for (B, H, S): fp32 delta and scaled LSE
 * (8*B*H*S bytes, rounded up to 256), then the row terms -LSE*log2(e)/scale2
 * and -delta in fp32 (8*B*H*ceil32(S) bytes, rounded up to 256). */
size_t fa2_bwd_workspace_bytes(int32_t B, int32_t H, int32_t S);

int fa2_bwd_f16(const fa2_bwd_params *p, int32_t mode, void *workspace,
                size_t workspace_bytes, void *stream);

/* Allocation-free backward: fa2_bwd_f16 (same modes, same kernels, same
 * results bit for bit) with no workspace argument.  Its workspace is scratch
 * memory inside the library: a device array of FA2_BWD_SCRATCH_MAX_BYTES that
 * every GPU the library runs on holds from the first use until the process
 * ends.  The call allocates nothing and frees nothing, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); the caller still provides inputs and outputs.
 *   - Size limit: fa2_bwd_noalloc_scratch_bytes(B, H, S) (delta, scaled LSE and
 *     the row terms: about 16*B*H*S bytes, the same as fa2_bwd_workspace_bytes)
 *     must not exceed FA2_BWD_SCRATCH_MAX_BYTES, else FA2_ERR_WORKSPACE.
 *   - Set-up: the device address of the array is looked up once per device, on
 *     the first call with that device current (a symbol lookup that may load the
 *     library's code object; it allocates nothing).  A caller that captures the
 *     call into a HIP graph makes one call on that device before capturing.
 *   - Sharing: all calls on one GPU share that GPU's array, which keeps the last
 *     call's contents.  Calls that overlap in time on one GPU (several streams
 *     or host threads) race on it and must be serialised by the caller.  Mode 4
 *     reads the delta an earlier mode 1 or 2 call left there, so that pair must
 *     run back to back on one stream with no other call in between.
 * No counterpart in the reference; for callers that cannot allocate. */
#define FA2_BWD_SCRATCH_MAX_BYTES (32u << 20)
size_t fa2_bwd_noalloc_scratch_bytes(int32_t B, int32_t H, int32_t S);
int fa2_bwd_f16_noalloc(const fa2_bwd_params *p, int32_t mode, void *stream);

/* Fused rotary embedding on q and k (head_dim 64), fp32 arithmetic with one
 * fp16 rounding, no fused multiply-add (bitwise equal to the eager fp32 path
 * followed by .half()):
 *   forward : out[d] = x[d]*cos[d] + r[d]*sin[d],  r[d] = -x[d+32] (d<32),
 *                                                       x[d-32]  (d>=32)
 *   backward: gx[d]  = g[d]*cos[d] + t[d],         t[d] = +g[d+32]*sin[d+32] (d<32),
 *                                                       -g[d-32]*sin[d-32] (d>=32)
 * cos/sin are fp32 [S,64] with row stride cs_stride/sn_stride.
 * Replaces fastops::rope_fwd / rope_bwd
 *   (reference @ None: csrc/flash_attn_v100/fast_ops.cu:31-216).
 * q/k/outputs need 4-byte alignment and even strides only. */
typedef struct fa2_rope_params {
    const void *q, *k;              /* fp16 [B,H,S,64] inputs (grads in bwd)   */
    void *qo, *ko;                  /* fp16 [B,H,S,64] outputs                 */
    const float *cos, *sin;         /* fp32 [S,64]                             */
    int64_t q_stride[3], k_stride[3], qo_stride[3], ko_stride[3];
    int64_t cs_stride, sn_stride;
    int32_t B, H, S, D;
} fa2_rope_params;

int fa2_rope_f16(const fa2_rope_params *p, int32_t backward, void *stream);

/* Human-readable text for a status code, and the detail message of the last
 * failing call on this host thread ("" if none). */
const char *fa2_status_string(int status);
const char *fa2_last_error(void);

/* Library version string and the gfx target the kernels were built for. */
const char *fa2_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA2_MI355X_H */
