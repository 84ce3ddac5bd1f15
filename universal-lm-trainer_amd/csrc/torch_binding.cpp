// torch_binding.cpp -- thin PyTorch-ROCm extension over the C ABI.
//
// Exposes the reference's four extension ops with their signatures and
// output conventions (reference @ None: csrc/flash_attn_v100/flash_attn_v100.cu:386-397):
//   fa_fwd(q, k, v, dropout_p, causal, softmax_scale, seed)            -> [o, lse]
// plus fa_fwd_mask (same arguments) -> [o, lse, mask]: with dropout also the
// keep-bit words (int32, fa2_dropout_mask_bytes[_causal]), for fa_bwd(..., mask=)
// to read instead of hashing again (identical gradients);
// plus, for inference callers (no reference counterpart; fa2_fwd_kv_f16):
//   fa_fwd_kv(q, k, v, causal, softmax_scale, causal_offset, nsplit=0)  -> [o, lse]
// with k, v of their own sequence length and key j visible to query i iff
// j <= i + causal_offset when causal; nsplit slices of the key range
// (fa2_fwd_kv_split_f16, 0 = chosen here so the grid fills the GPU).
//   fa_bwd(q, k, v, o, lse, do, dropout_p, causal, softmax_scale, seed,
//          mode=7, mask=None)                                           -> [dq, dk, dv]
//   rope_fwd(q, k, cos, sin)                                            -> [qo, ko]
//   rope_bwd(dqo, dko, cos, sin, q, k)                                  -> [dq, dk]
// Inputs are borrowed with their strides; outputs and the backward's
// workspace come from the torch caching allocator on q's device (fa_fwd's O
// follows q's memory order, see fa_fwd); launches go to the current stream
// with no host synchronisation.  A nonzero status from
// the C ABI becomes a RuntimeError carrying the library's message.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <algorithm>
#include <vector>

#include "../../include/fa2_mi355x.h"

namespace {

void *current_stream(const torch::Tensor &t) {
    return reinterpret_cast<void *>(at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

void check_status(int rc, const char *op) {
    TORCH_CHECK(rc == FA2_OK, op, ": ", fa2_status_string(rc), ": ", fa2_last_error());
}

// The C ABI takes B, H, S as int32.
void check_dims(const torch::Tensor &t, const char *op) {
    TORCH_CHECK(t.size(0) <= INT32_MAX && t.size(1) <= INT32_MAX && t.size(2) <= INT32_MAX, op,
                ": B, H and S must fit in int32");
}

void strides3(const torch::Tensor &t, int64_t out[3]) {
    out[0] = t.stride(0);
    out[1] = t.stride(1);
    out[2] = t.stride(2);
}

// Same contract checks as the reference's check_fwd (flash_attn_v100.cu:314-335).
void check_qkv(const torch::Tensor &q, const torch::Tensor &k, const torch::Tensor &v) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "inputs must be on the GPU");
    TORCH_CHECK(q.dtype() == torch::kHalf && k.dtype() == torch::kHalf && v.dtype() == torch::kHalf,
                "only fp16 supported");
    TORCH_CHECK(q.dim() == 4, "q must be (B,H,S,D)");
    TORCH_CHECK(q.size(3) == 64, "head_dim must be 64");
    TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(), "q/k/v shape mismatch");
    TORCH_CHECK(k.device() == q.device() && v.device() == q.device(), "q/k/v device mismatch");
    TORCH_CHECK(q.stride(3) == 1 && k.stride(3) == 1 && v.stride(3) == 1, "last dim must be contiguous");
}

// The forward through fa2_fwd_kv_f16 (s_k = k's length); fa_fwd is the square case.
std::vector<torch::Tensor> fwd_impl(const torch::Tensor &q, const torch::Tensor &k, const torch::Tensor &v,
                                    double dropout_p, bool causal, double softmax_scale, int64_t seed,
                                    int64_t causal_offset, const char *op, int64_t nsplit = 1,
                                    bool want_mask = false) {
    check_dims(q, op);
    at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    const int64_t B = q.size(0), H = q.size(1), S = q.size(2);
    // O follows q's memory order the way an eager elementwise output would:
    // for the (B,S,H,D) layout train.py produces (q.stride(1) == 64,
    // q.stride(2) >= H*64) O is stored as [B,S,H,64] and returned as the
    // (B,H,S,64) view, so the caller's transpose(1,2).contiguous() is free;
    // otherwise O is contiguous (B,H,S,64) as in the reference
    // (flash_attn_v100.cu:342).
    const bool bshd = q.stride(1) == 64 && q.stride(2) >= H * 64 && H > 1;
    auto o = bshd ? torch::empty({B, S, H, 64}, q.options()).transpose(1, 2)
                  : torch::empty({B, H, S, 64}, q.options());
    auto lse = torch::empty({B, H, S}, q.options().dtype(torch::kFloat));
    fa2_fwd_params p;
    memset(&p, 0, sizeof(p));
    p.q = q.data_ptr();
    p.k = k.data_ptr();
    p.v = v.data_ptr();
    p.o = o.data_ptr();
    p.lse = lse.data_ptr<float>();
    strides3(q, p.q_stride);
    strides3(k, p.k_stride);
    strides3(v, p.v_stride);
    strides3(o, p.o_stride);
    p.lse_stride[0] = lse.stride(0);
    p.lse_stride[1] = lse.stride(1);
    p.B = (int32_t)B;
    p.H = (int32_t)H;
    p.S = (int32_t)S;
    p.D = 64;
    p.softmax_scale = (float)softmax_scale;
    p.dropout_p = (float)dropout_p;
    p.seed = (uint32_t)seed;
    p.causal = causal ? 1 : 0;
    TORCH_CHECK(k.size(2) <= INT32_MAX && causal_offset >= INT32_MIN && causal_offset <= INT32_MAX,
                op, ": key length / causal offset out of range");
    if (want_mask) {   // square forward (fa2_fwd_f16), which alone writes keep bits (none without dropout)
        const size_t mask_bytes = causal ? fa2_dropout_mask_bytes_causal(p.B, p.H, p.S)
                                         : fa2_dropout_mask_bytes(p.B, p.H, p.S);
        auto mask = torch::empty({dropout_p > 0.0 ? (int64_t)(mask_bytes / 4) : 0},
                                 q.options().dtype(torch::kInt));
        p.dropout_mask = dropout_p > 0.0 ? reinterpret_cast<uint32_t *>(mask.data_ptr()) : nullptr;
        p.dropout_mask_bytes = (size_t)mask.numel() * 4;
        check_status(fa2_fwd_f16(&p, current_stream(q)), op);
        return {o, lse, mask};
    }
    if (nsplit <= 1) {
        check_status(fa2_fwd_kv_f16(&p, (int32_t)k.size(2), (int32_t)causal_offset, current_stream(q)), op);
    } else {
        const size_t bytes = fa2_fwd_kv_workspace_bytes(p.B, p.H, p.S, (int32_t)nsplit);
        auto ws = torch::empty({(int64_t)(bytes / 4) + 4}, q.options().dtype(torch::kFloat));
        check_status(fa2_fwd_kv_split_f16(&p, (int32_t)k.size(2), (int32_t)causal_offset, (int32_t)nsplit,
                                          ws.data_ptr(), ws.numel() * 4, current_stream(q)),
                     op);
    }
    return {o, lse};
}

std::vector<torch::Tensor> fa_fwd(torch::Tensor q, torch::Tensor k, torch::Tensor v, double dropout_p, bool causal,
                                  double softmax_scale, int64_t seed) {
    check_qkv(q, k, v);
    return fwd_impl(q, k, v, dropout_p, causal, softmax_scale, seed, 0, "fa_fwd");
}

std::vector<torch::Tensor> fa_fwd_mask(torch::Tensor q, torch::Tensor k, torch::Tensor v, double dropout_p,
                                       bool causal, double softmax_scale, int64_t seed) {
    check_qkv(q, k, v);
    return fwd_impl(q, k, v, dropout_p, causal, softmax_scale, seed, 0, "fa_fwd_mask", 1, true);
}

// Key slices for a grid of `wgs` workgroups over `tiles` 64-key tiles: about
// 384 workgroups in all (1.5 per CU) with at least 8 tiles per slice -- the
// best of a sweep over decode (S_q = 1, S_k = 4K..16K, B*H = 12..96) and
// chunks (S_q = 128..512); more slices lose to each slice's fixed costs.
int64_t auto_nsplit(int64_t wgs, int64_t tiles) {
    return std::max<int64_t>(1, std::min<int64_t>(384 / wgs, tiles / 8));
}

// Decode (one query, the VALU kernel, four waves per workgroup each taking a
// quarter of its slice): about 192 workgroups and at least 1024 keys per
// slice -- the best of a sweep over B*H = 12..384 and S_k = 1K..16K.
int64_t auto_nsplit_decode(int64_t bh, int64_t s_k) {
    return std::max<int64_t>(1, std::min<int64_t>((192 + bh - 1) / bh, s_k / 1024));
}

std::vector<torch::Tensor> fa_fwd_kv(torch::Tensor q, torch::Tensor k, torch::Tensor v, bool causal,
                                     double softmax_scale, int64_t causal_offset, int64_t nsplit) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "inputs must be on the GPU");
    TORCH_CHECK(q.dtype() == torch::kHalf && k.dtype() == torch::kHalf && v.dtype() == torch::kHalf,
                "only fp16 supported");
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "q, k, v must be (B,H,S,D)");
    TORCH_CHECK(q.size(3) == 64 && k.size(3) == 64 && v.size(3) == 64, "head_dim must be 64");
    TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(1) == q.size(1),
                "k/v must be (B,H,S_k,64) with q's B and H");
    TORCH_CHECK(k.size(2) >= 1, "empty key sequence");
    TORCH_CHECK(k.device() == q.device() && v.device() == q.device(), "q/k/v device mismatch");
    TORCH_CHECK(q.stride(3) == 1 && k.stride(3) == 1 && v.stride(3) == 1, "last dim must be contiguous");
    TORCH_CHECK(nsplit >= 0 && nsplit <= 1024, "nsplit must be 0 (automatic) .. 1024");
    if (nsplit == 0 && q.numel() == 0) nsplit = 1;   // nothing to run (and no grid to size)
    if (nsplit == 0)
        nsplit = q.size(2) == 1 ? auto_nsplit_decode(q.size(0) * q.size(1), k.size(2))
                                : auto_nsplit((q.size(2) + 127) / 128 * q.size(0) * q.size(1), (k.size(2) + 63) / 64);
    return fwd_impl(q, k, v, 0.0, causal, softmax_scale, 0, causal_offset, "fa_fwd_kv", nsplit);
}

std::vector<torch::Tensor> fa_bwd(torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor o,
                                  torch::Tensor lse, torch::Tensor do_, double dropout_p, bool causal,
                                  double softmax_scale, int64_t seed, int64_t mode,
                                  c10::optional<torch::Tensor> mask) {
    check_qkv(q, k, v);
    TORCH_CHECK(o.sizes() == q.sizes() && do_.sizes() == q.sizes(), "o/do shape mismatch");
    TORCH_CHECK(o.dtype() == torch::kHalf && do_.dtype() == torch::kHalf, "o/do must be fp16");
    TORCH_CHECK(lse.dtype() == torch::kFloat && lse.dim() == 3 && lse.size(0) == q.size(0) &&
                    lse.size(1) == q.size(1) && lse.size(2) == q.size(2),
                "lse must be fp32 (B,H,S)");
    // The reference tests bits 1, 2 and 4 of mode and ignores the rest
    // (flash_attn_v100_bwd.cu:476-502).
    TORCH_CHECK(mode >= 0, "mode must be a non-negative bit mask");
    check_dims(q, "fa_bwd");
    if (mask && dropout_p > 0.0) {
        TORCH_CHECK(mask->is_cuda() && mask->device() == q.device() && mask->dtype() == torch::kInt &&
                        mask->is_contiguous(),
                    "fa_bwd: mask must be the contiguous int32 words fa_fwd_mask returned");
        const int32_t B = (int32_t)q.size(0), H = (int32_t)q.size(1), S = (int32_t)q.size(2);
        TORCH_CHECK((size_t)mask->numel() * 4 ==
                        (causal ? fa2_dropout_mask_bytes_causal(B, H, S) : fa2_dropout_mask_bytes(B, H, S)),
                    "fa_bwd: mask size does not match (B, H, S, causal)");
    }
    at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    // The kernels take any (b,h,s) strides; only rows must be contiguous and
    // 16-byte aligned.  lse must have unit stride along s.
    auto o_c = (o.stride(3) == 1 && o.stride(2) % 8 == 0 && o.stride(1) % 8 == 0 && o.stride(0) % 8 == 0)
                   ? o
                   : o.contiguous();
    auto do_c = (do_.stride(3) == 1 && do_.stride(2) % 8 == 0 && do_.stride(1) % 8 == 0 && do_.stride(0) % 8 == 0)
                    ? do_
                    : do_.contiguous();
    auto lse_c = lse.stride(2) == 1 ? lse : lse.contiguous();
    const int64_t B = q.size(0), H = q.size(1), S = q.size(2);
    auto dq = torch::empty({B, H, S, 64}, q.options());
    auto dk = torch::empty({B, H, S, 64}, q.options());
    auto dv = torch::empty({B, H, S, 64}, q.options());
    auto ws = torch::empty({(int64_t)fa2_bwd_workspace_bytes((int32_t)B, (int32_t)H, (int32_t)S) / 4 + 64},
                           q.options().dtype(torch::kFloat));
    fa2_bwd_params p;
    memset(&p, 0, sizeof(p));
    p.q = q.data_ptr();
    p.k = k.data_ptr();
    p.v = v.data_ptr();
    p.o = o_c.data_ptr();
    p.dout = do_c.data_ptr();
    p.lse = lse_c.data_ptr<float>();
    p.dq = dq.data_ptr();
    p.dk = dk.data_ptr();
    p.dv = dv.data_ptr();
    strides3(q, p.q_stride);
    strides3(k, p.k_stride);
    strides3(v, p.v_stride);
    strides3(o_c, p.o_stride);
    strides3(do_c, p.do_stride);
    strides3(dq, p.dq_stride);
    strides3(dk, p.dk_stride);
    strides3(dv, p.dv_stride);
    p.lse_stride[0] = lse_c.stride(0);
    p.lse_stride[1] = lse_c.stride(1);
    p.B = (int32_t)B;
    p.H = (int32_t)H;
    p.S = (int32_t)S;
    p.D = 64;
    p.softmax_scale = (float)softmax_scale;
    p.dropout_p = (float)dropout_p;
    p.seed = (uint32_t)seed;
    p.causal = causal ? 1 : 0;
    if (mask && dropout_p > 0.0) {
        p.dropout_mask = reinterpret_cast<const uint32_t *>(mask->data_ptr());
        p.dropout_mask_bytes = (size_t)mask->numel() * 4;
    }
    // The workspace is fresh each call, so a dK/dV-only request also computes
    // delta (the reference would read an uninitialised buffer there).
    int32_t m = (int32_t)(mode & 7);
    if ((m & 4) && !(m & 3)) m |= 1;
    check_status(fa2_bwd_f16(&p, m, ws.data_ptr(), (size_t)ws.numel() * 4, current_stream(q)), "fa_bwd");
    return {dq, dk, dv};
}

// RoPE outputs get the memory order the eager expression x*cos + rotate_half(x)*sin
// would give them (reference @ None: fast_ops.cu:142-150): an input that fills
// its storage span keeps its own layout; a head-interleaved view (q or k of
// the fused qkv projection: heads adjacent, positions H*64 or more apart)
// becomes a packed (B, S, H, 64) tensor; any other view a packed (B, H, S, 64) one.
std::vector<int64_t> rope_out_strides(const torch::Tensor &x) {
    if (x.is_non_overlapping_and_dense()) return x.strides().vec();
    const int64_t H = x.size(1), S = x.size(2), D = x.size(3);
    const bool heads_inner = x.stride(1) == D && x.stride(2) >= H * D;
    if (heads_inner) return {S * H * D, D, H * D, 1};
    return {H * S * D, S * D, D, 1};
}

// Eligibility of the fused RoPE ops, each failure with its own message.
void rope_check(const torch::Tensor &q, const torch::Tensor &k, const torch::Tensor &cos, const torch::Tensor &sin) {
    auto need = [](bool ok, const char *what) { TORCH_CHECK(ok, "fused RoPE: ", what); };
    need(q.is_cuda() && k.is_cuda() && k.device() == q.device(), "q and k must be on one GPU");
    need(q.dtype() == torch::kHalf && k.dtype() == torch::kHalf, "q and k must be fp16");
    need(q.dim() == 4 && q.size(3) == 64 && q.sizes() == k.sizes(), "q and k must both be [B, H, S, 64]");
    need(q.stride(3) == 1 && k.stride(3) == 1, "the head dimension of q and k must be unit-stride");
    need(cos.is_cuda() && sin.is_cuda() && cos.device() == q.device() && sin.device() == q.device(),
         "cos and sin must be on q's GPU");
    need(cos.dtype() == torch::kFloat && sin.dtype() == torch::kFloat, "cos and sin must be fp32");
    need(cos.dim() == 2 && cos.size(0) == q.size(2) && cos.size(1) == 64 && cos.sizes() == sin.sizes(),
         "cos and sin must be [S, 64] with q's S");
    need(cos.stride(1) == 1 && sin.stride(1) == 1, "cos and sin rows must be unit-stride");
}

std::vector<torch::Tensor> rope_run(const torch::Tensor &x, const torch::Tensor &y, const torch::Tensor &cos,
                                    const torch::Tensor &sin, const torch::Tensor &shape_q,
                                    const torch::Tensor &shape_k, bool backward) {
    check_dims(x, backward ? "rope_bwd" : "rope_fwd");
    at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    auto qo = torch::empty_strided(shape_q.sizes(), rope_out_strides(shape_q), shape_q.options());
    auto ko = torch::empty_strided(shape_k.sizes(), rope_out_strides(shape_k), shape_k.options());
    fa2_rope_params p;
    memset(&p, 0, sizeof(p));
    p.q = x.data_ptr();
    p.k = y.data_ptr();
    p.qo = qo.data_ptr();
    p.ko = ko.data_ptr();
    p.cos = cos.data_ptr<float>();
    p.sin = sin.data_ptr<float>();
    strides3(x, p.q_stride);
    strides3(y, p.k_stride);
    strides3(qo, p.qo_stride);
    strides3(ko, p.ko_stride);
    p.cs_stride = cos.stride(0);
    p.sn_stride = sin.stride(0);
    p.B = (int32_t)x.size(0);
    p.H = (int32_t)x.size(1);
    p.S = (int32_t)x.size(2);
    p.D = 64;
    check_status(fa2_rope_f16(&p, backward ? 1 : 0, current_stream(x)), backward ? "rope_bwd" : "rope_fwd");
    return {qo, ko};
}

std::vector<torch::Tensor> rope_fwd(torch::Tensor q, torch::Tensor k, torch::Tensor cos, torch::Tensor sin) {
    rope_check(q, k, cos, sin);
    return rope_run(q, k, cos, sin, q, k, false);
}

std::vector<torch::Tensor> rope_bwd(torch::Tensor dqo, torch::Tensor dko, torch::Tensor cos, torch::Tensor sin,
                                    torch::Tensor q, torch::Tensor k) {
    rope_check(q, k, cos, sin);
    rope_check(dqo, dko, cos, sin);   // the incoming gradients obey the same rules
    TORCH_CHECK(dqo.sizes() == q.sizes(), "fused RoPE backward: gradients must have q's shape");
    return rope_run(dqo, dko, cos, sin, q, k, true);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("fa_fwd", &fa_fwd, "FA2 forward (gfx950 MFMA)");
    m.def("fa_fwd_mask", &fa_fwd_mask, "FA2 forward that also returns the dropout keep-bit words");
    m.def("fa_fwd_kv", &fa_fwd_kv, "FA2 forward, k/v of their own length (inference)", pybind11::arg("q"),
          pybind11::arg("k"), pybind11::arg("v"), pybind11::arg("causal"), pybind11::arg("softmax_scale"),
          pybind11::arg("causal_offset"), pybind11::arg("nsplit") = 0);
    m.def("fa_bwd", &fa_bwd, "FA2 backward (gfx950 MFMA)", pybind11::arg("q"), pybind11::arg("k"),
          pybind11::arg("v"), pybind11::arg("o"), pybind11::arg("lse"), pybind11::arg("do"),
          pybind11::arg("dropout_p"), pybind11::arg("causal"), pybind11::arg("softmax_scale"),
          pybind11::arg("seed"), pybind11::arg("mode") = 7, pybind11::arg("mask") = pybind11::none());
    m.def("rope_fwd", &rope_fwd, "fused RoPE forward");
    m.def("rope_bwd", &rope_bwd, "fused RoPE backward");
    m.def("version", []() { return std::string(fa2_version()); });
}
