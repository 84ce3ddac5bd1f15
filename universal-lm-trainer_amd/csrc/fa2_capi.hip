// fa2_capi.hip -- the C ABI (include/fa2_mi355x.h): argument validation,
// kernel-argument packing and launches.  Allocates nothing and never
// synchronises; its only state is a thread-local error message, a per-device
// cache of the compute-unit count, and the per-device scratch array of the
// allocation-free backward.
#include <float.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "../../include/fa2_mi355x.h"
#include "fa2_kernels.h"

namespace {

thread_local char g_err[512] = {0};

int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest element offset reachable by a [B,H,S,64] view with these strides
// must fit int64 and each stride must keep 16-byte row alignment.
int check_tensor(const char *name, const void *ptr, const int64_t st[3], int32_t B, int32_t H, int32_t S,
                 bool vec16) {
    if (!ptr) return fail(FA2_ERR_NULL_POINTER, "%s is NULL", name);
    for (int i = 0; i < 3; ++i) {
        if (st[i] < 0) return fail(FA2_ERR_BAD_SHAPE, "%s stride[%d] = %lld is negative", name, i, (long long)st[i]);
        if (vec16 && (st[i] % 8) != 0)
            return fail(FA2_ERR_MISALIGNED, "%s stride[%d] = %lld is not a multiple of 8 elements", name, i,
                        (long long)st[i]);
        if (!vec16 && (st[i] % 2) != 0)
            return fail(FA2_ERR_MISALIGNED, "%s stride[%d] = %lld is odd", name, i, (long long)st[i]);
    }
    // Kernels address a 64-row tile with 32-bit byte offsets from its first row.
    if (st[2] >= (1 << 24))
        return fail(FA2_ERR_BAD_SHAPE, "%s sequence stride %lld is not below 2^24 elements", name, (long long)st[2]);
    if (vec16 && !aligned16(ptr)) return fail(FA2_ERR_MISALIGNED, "%s is not 16-byte aligned", name);
    if (!vec16 && (reinterpret_cast<uintptr_t>(ptr) & 3u))
        return fail(FA2_ERR_MISALIGNED, "%s is not 4-byte aligned", name);
    const double span = (double)(B - 1) * st[0] + (double)(H - 1) * st[1] + (double)(S - 1) * st[2] + 64.0;
    if (span > 9.0e18) return fail(FA2_ERR_BAD_SHAPE, "%s spans more than 2^63 elements", name);
    return FA2_OK;
}

int check_shape(int32_t B, int32_t H, int32_t S, int32_t D, int per_wg) {
    if (B < 0 || H < 0 || S < 0) return fail(FA2_ERR_BAD_SHAPE, "negative size B=%d H=%d S=%d", B, H, S);
    if (D != FA2_HEAD_DIM) return fail(FA2_ERR_BAD_SHAPE, "head dim %d unsupported (must be 64)", D);
    const double grid = (double)B * H * ((S + per_wg - 1) / per_wg + 1);
    if (grid > 2147483647.0 || (double)B * H * S > 2147483647.0)
        return fail(FA2_ERR_BAD_SHAPE, "B*H*S = %.0f exceeds the int32 grid limit", (double)B * H * S);
    return FA2_OK;
}

int check_scale_dropout(float scale, float p) {
    if (!isfinite(scale)) return fail(FA2_ERR_BAD_ARGUMENT, "softmax_scale %g is not finite", (double)scale);
    if (!(p >= 0.f && p < 1.f)) return fail(FA2_ERR_BAD_ARGUMENT, "dropout_p %g outside [0, 1)", (double)p);
    return FA2_OK;
}

float scale2_of(float scale) {
    const float s2 = fabsf(scale) * 1.4426950408889634f;  // log2(e)
    return s2 < FLT_MIN ? FLT_MIN : s2;
}

// The keep-bit words are moved in 16-byte transfers and cover every (b, h)
// at fixed offsets; without dropout they are not touched.
int check_mask(const void *mask, size_t bytes, int32_t B, int32_t H, int32_t S, float p, int32_t causal) {
    if (!mask || !(p > 0.f)) return FA2_OK;
    if (reinterpret_cast<uintptr_t>(mask) & 15u) return fail(FA2_ERR_MISALIGNED, "dropout_mask is not 16-byte aligned");
    const size_t need = causal ? fa2_dropout_mask_bytes_causal(B, H, S) : fa2_dropout_mask_bytes(B, H, S);
    if (bytes < need) return fail(FA2_ERR_WORKSPACE, "dropout_mask needs %zu bytes, got %zu", need, bytes);
    return FA2_OK;
}

}  // namespace

namespace fa2 {
int device_cus() {
    // Relaxed atomics: racing first calls on several host threads each store
    // the same value.
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}
}  // namespace fa2

extern "C" {

// keep iff (hash >> 8) * 2^-24 >= p  <=>  (hash >> 8) >= ceil(p * 2^24): p * 2^24
// is exact in fp32 (a power-of-two scaling) and so is its ceiling.
uint32_t fa2_dropout_threshold(float p) {
    if (!(p > 0.f)) return 0;
    if (!(p < 1.f)) return 1u << 24;
    return (uint32_t)ceilf(p * 16777216.0f);
}

const char *fa2_status_string(int status) {
    switch (status) {
        case FA2_OK: return "ok";
        case FA2_ERR_NULL_POINTER: return "null pointer";
        case FA2_ERR_BAD_SHAPE: return "bad shape";
        case FA2_ERR_MISALIGNED: return "misaligned pointer or stride";
        case FA2_ERR_BAD_ARGUMENT: return "bad argument";
        case FA2_ERR_WORKSPACE: return "workspace missing or too small";
        case FA2_ERR_LAUNCH: return "kernel launch failed";
        default: return "unknown status";
    }
}

const char *fa2_last_error(void) { return g_err; }

const char *fa2_version(void) { return "fa2_mi355x 0.1 (gfx950, fp16 MFMA 32x32x16)"; }

static size_t kv_part_bytes(int32_t B, int32_t H, int32_t S, int32_t nsplit) {
    return (size_t)nsplit * B * H * S * (FA2_HEAD_DIM + 2) * sizeof(float);
}

size_t fa2_dropout_mask_bytes(int32_t B, int32_t H, int32_t S) {
    if (B <= 0 || H <= 0 || S <= 0) return 0;
    const size_t tiles = 2 * (((size_t)S + 127) / 128), rows = ((size_t)S + 255) & ~(size_t)255;
    return (size_t)B * H * tiles * 2 * rows * sizeof(uint32_t);
}

// Causal: 128-key block j keeps runs of R - 128 j words (4 runs: 2 tiles x 2 halves).
size_t fa2_dropout_mask_bytes_causal(int32_t B, int32_t H, int32_t S) {
    if (B <= 0 || H <= 0 || S <= 0) return 0;
    const size_t J = ((size_t)S + 127) / 128, R = ((size_t)S + 255) & ~(size_t)255;
    return (size_t)B * H * (4 * J * R - 256 * J * (J - 1)) * sizeof(uint32_t);
}

size_t fa2_fwd_kv_workspace_bytes(int32_t B, int32_t H, int32_t S, int32_t nsplit) {
    if (B <= 0 || H <= 0 || S <= 0 || nsplit <= 1) return 0;
    return kv_part_bytes(B, H, S, nsplit);
}

// The forward over s_k key rows with key j visible to query i iff
// j <= i + coff (causal); fa2_fwd_f16 is s_k = S, coff = 0.  nsplit > 1
// cuts the key range into slices whose partial results (in the workspace)
// a second kernel merges.
// `inference`: the fa2_fwd_kv_* entry points, where one query without dropout
// takes the decode kernel.
static int fwd_common(const fa2_fwd_params *p, int32_t s_k, int32_t coff, void *stream, bool inference,
                      int32_t nsplit = 1, void *workspace = nullptr, size_t workspace_bytes = 0) {
    if (!p) return fail(FA2_ERR_NULL_POINTER, "params is NULL");
    if (nsplit < 1 || nsplit > 1024) return fail(FA2_ERR_BAD_ARGUMENT, "nsplit %d outside 1..1024", nsplit);
    int rc = check_shape(p->B, p->H, p->S, p->D, 256);
    if (rc) return rc;
    if ((rc = check_scale_dropout(p->softmax_scale, p->dropout_p))) return rc;
    if (inference && p->dropout_mask)
        return fail(FA2_ERR_BAD_ARGUMENT, "dropout_mask must be NULL for the fa2_fwd_kv_* entry points");
    if ((int64_t)p->B * p->H * p->S == 0) return FA2_OK;
    if (s_k < 1 || (double)p->B * p->H * s_k > 2147483647.0)
        return fail(FA2_ERR_BAD_SHAPE, "key length %d outside 1 .. 2^31 / (B*H)", s_k);
    if (coff < -(1 << 30) || coff > (1 << 30))
        return fail(FA2_ERR_BAD_ARGUMENT, "causal offset %d outside +-2^30", coff);
    if (nsplit > 1) {
        // one workgroup per (128-query block, slice, b*h); one per (slice, b*h) for decode
        if ((double)p->B * p->H * ((p->S + 127) / 128) * nsplit > 2147483647.0)
            return fail(FA2_ERR_BAD_SHAPE, "B*H*ceil(S/128)*nsplit = %.0f exceeds the int32 grid limit",
                        (double)p->B * p->H * ((p->S + 127) / 128) * nsplit);
        const size_t need = kv_part_bytes(p->B, p->H, p->S, nsplit);
        if (!workspace || workspace_bytes < need)
            return fail(FA2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : 0);
        if (reinterpret_cast<uintptr_t>(workspace) & 15u)
            return fail(FA2_ERR_MISALIGNED, "workspace is not 16-byte aligned");
    }
    if ((rc = check_tensor("q", p->q, p->q_stride, p->B, p->H, p->S, true))) return rc;
    if ((rc = check_tensor("k", p->k, p->k_stride, p->B, p->H, s_k, true))) return rc;
    if ((rc = check_tensor("v", p->v, p->v_stride, p->B, p->H, s_k, true))) return rc;
    if ((rc = check_tensor("o", p->o, p->o_stride, p->B, p->H, p->S, false))) return rc;
    if (!aligned16(p->o) || (p->o_stride[0] | p->o_stride[1] | p->o_stride[2]) % 4)
        return fail(FA2_ERR_MISALIGNED, "o needs 16-byte base alignment and strides that are multiples of 4");
    if (!p->lse) return fail(FA2_ERR_NULL_POINTER, "lse is NULL");
    if (reinterpret_cast<uintptr_t>(p->lse) & 3u) return fail(FA2_ERR_MISALIGNED, "lse is not 4-byte aligned");
    if (p->lse_stride[0] < 0 || p->lse_stride[1] < 0) return fail(FA2_ERR_BAD_SHAPE, "negative lse stride");
    if ((rc = check_mask(p->dropout_mask, p->dropout_mask_bytes, p->B, p->H, p->S, p->dropout_p, p->causal))) return rc;

    fa2::FwdArgs a;
    a.q = static_cast<const _Float16 *>(p->q);
    a.k = static_cast<const _Float16 *>(p->k);
    a.v = static_cast<const _Float16 *>(p->v);
    a.o = static_cast<_Float16 *>(p->o);
    a.lse = p->lse;
    a.qsb = p->q_stride[0]; a.qsh = p->q_stride[1]; a.qss = p->q_stride[2];
    a.ksb = p->k_stride[0]; a.ksh = p->k_stride[1]; a.kss = p->k_stride[2];
    a.vsb = p->v_stride[0]; a.vsh = p->v_stride[1]; a.vss = p->v_stride[2];
    a.osb = p->o_stride[0]; a.osh = p->o_stride[1]; a.oss = p->o_stride[2];
    a.lsb = p->lse_stride[0]; a.lsh = p->lse_stride[1];
    a.B = p->B; a.H = p->H; a.S = p->S;
    a.Sk = s_k;
    a.coff = coff;
    const int32_t tiles = (s_k + 63) / 64;
    a.nsplit = nsplit;
    a.split_keys = 64 * ((tiles + nsplit - 1) / nsplit);
    a.part_o = nsplit > 1 ? static_cast<float *>(workspace) : nullptr;
    a.part_ml = nsplit > 1 ? a.part_o + (size_t)nsplit * p->B * p->H * p->S * FA2_HEAD_DIM : nullptr;
    a.scale2 = scale2_of(p->softmax_scale);
    a.negate = p->softmax_scale < 0.f;
    a.seed = p->seed;
    a.drop_thr = fa2_dropout_threshold(p->dropout_p);
    a.inv_keep = 1.f / (1.f - p->dropout_p);
    const bool causal = p->causal != 0, dropout = p->dropout_p > 0.f;
    a.drop_mask = dropout ? p->dropout_mask : nullptr;
    a.hgroup = 0;
    const hipStream_t st = (hipStream_t)stream;
    const hipError_t e = (inference && p->S == 1 && !dropout) ? fa2::launch_fwd_decode(a, causal, st)
                         : nsplit > 1                         ? fa2::launch_fwd_split(a, causal, dropout, st)
                                                              : fa2::launch_fwd(a, causal, dropout, st);
    if (e != hipSuccess) return fail(FA2_ERR_LAUNCH, "forward launch: %s", hipGetErrorString(e));
    return FA2_OK;
}

int fa2_fwd_f16(const fa2_fwd_params *p, void *stream) {
    g_err[0] = 0;
    return fwd_common(p, p ? p->S : 0, 0, stream, false);
}

int fa2_fwd_kv_f16(const fa2_fwd_params *p, int32_t s_k, int32_t causal_offset, void *stream) {
    g_err[0] = 0;
    return fwd_common(p, s_k, causal_offset, stream, true);
}

int fa2_fwd_kv_split_f16(const fa2_fwd_params *p, int32_t s_k, int32_t causal_offset, int32_t nsplit,
                         void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    return fwd_common(p, s_k, causal_offset, stream, true, nsplit, workspace, workspace_bytes);
}

// Workspace: fp32 delta and log2-scaled LSE, [B*H*S] each (rounded up to 256
// bytes), then the per-row terms -LSE*log2(e)/scale2 and -delta in fp32, 8
// bytes per query with S rounded up to 32 (rounded up to 256 bytes).
static size_t delta_bytes(int32_t B, int32_t H, int32_t S) {
    return ((size_t)B * H * S * 2 * sizeof(float) + 255) & ~(size_t)255;
}
static size_t terms_bytes(int32_t B, int32_t H, int32_t S) {
    return ((size_t)B * H * (((size_t)S + 31) & ~(size_t)31) * 8 + 255) & ~(size_t)255;
}

size_t fa2_bwd_workspace_bytes(int32_t B, int32_t H, int32_t S) {
    if (B <= 0 || H <= 0 || S <= 0) return 0;
    return delta_bytes(B, H, S) + terms_bytes(B, H, S);
}

// Checks of fa2_bwd_f16 that come before its workspace: status, or -1 when
// the call has nothing to do (empty problem or mode 0) and returns FA2_OK.
static int bwd_precheck(const fa2_bwd_params *p, int32_t mode) {
    if (!p) return fail(FA2_ERR_NULL_POINTER, "params is NULL");
    if (mode < 0 || mode > 7) return fail(FA2_ERR_BAD_ARGUMENT, "mode %d outside 0..7", mode);
    int rc = check_shape(p->B, p->H, p->S, p->D, 256);
    if (rc) return rc;
    if ((rc = check_scale_dropout(p->softmax_scale, p->dropout_p))) return rc;
    if ((int64_t)p->B * p->H * p->S == 0 || mode == 0) return -1;
    // The dK/dV pass reaches the LSE copy with a 32-bit byte offset from delta.
    if ((int64_t)p->B * p->H * p->S >= (int64_t)1 << 30)
        return fail(FA2_ERR_BAD_SHAPE, "B*H*S = %lld is not below 2^30", (long long)p->B * p->H * p->S);
    return FA2_OK;
}

// The backward on a workspace already checked to hold delta, the scaled LSE
// and the row terms.
static int bwd_run(const fa2_bwd_params *p, int32_t mode, void *workspace, void *stream) {
    int rc;
    const bool want_delta = mode & 1, want_dq = mode & 2, want_dkv = mode & 4;
    if ((rc = check_tensor("o", p->o, p->o_stride, p->B, p->H, p->S, true))) return rc;
    if ((rc = check_tensor("dout", p->dout, p->do_stride, p->B, p->H, p->S, true))) return rc;
    if (want_dq || want_dkv) {
        if ((rc = check_tensor("q", p->q, p->q_stride, p->B, p->H, p->S, true))) return rc;
        if ((rc = check_tensor("k", p->k, p->k_stride, p->B, p->H, p->S, true))) return rc;
        if ((rc = check_tensor("v", p->v, p->v_stride, p->B, p->H, p->S, true))) return rc;
        if (!p->lse) return fail(FA2_ERR_NULL_POINTER, "lse is NULL");
        if (reinterpret_cast<uintptr_t>(p->lse) & 3u) return fail(FA2_ERR_MISALIGNED, "lse is not 4-byte aligned");
        if (p->lse_stride[0] < 0 || p->lse_stride[1] < 0) return fail(FA2_ERR_BAD_SHAPE, "negative lse stride");
        if ((rc = check_mask(p->dropout_mask, p->dropout_mask_bytes, p->B, p->H, p->S, p->dropout_p, p->causal))) return rc;
    }
    struct Out { const char *name; void *ptr; const int64_t *st; };
    const Out outs[3] = {{"dq", p->dq, p->dq_stride}, {"dk", p->dk, p->dk_stride}, {"dv", p->dv, p->dv_stride}};
    for (int i = 0; i < 3; ++i) {
        if (i == 0 && !want_dq) continue;
        if (i > 0 && !want_dkv) continue;
        if ((rc = check_tensor(outs[i].name, outs[i].ptr, outs[i].st, p->B, p->H, p->S, false))) return rc;
        if (!aligned16(outs[i].ptr) || (outs[i].st[0] | outs[i].st[1] | outs[i].st[2]) % 4)
            return fail(FA2_ERR_MISALIGNED, "%s needs 16-byte base alignment and strides that are multiples of 4",
                        outs[i].name);
    }

    fa2::BwdArgs a;
    a.q = static_cast<const _Float16 *>(p->q);
    a.k = static_cast<const _Float16 *>(p->k);
    a.v = static_cast<const _Float16 *>(p->v);
    a.o = static_cast<const _Float16 *>(p->o);
    a.dout = static_cast<const _Float16 *>(p->dout);
    a.lse = p->lse;
    a.dq = static_cast<_Float16 *>(p->dq);
    a.dk = static_cast<_Float16 *>(p->dk);
    a.dv = static_cast<_Float16 *>(p->dv);
    a.delta = static_cast<float *>(workspace);
    a.lse2 = a.delta + (int64_t)p->B * p->H * p->S;
    a.rowterm = reinterpret_cast<float *>(static_cast<char *>(workspace) + delta_bytes(p->B, p->H, p->S));
    a.qsb = p->q_stride[0]; a.qsh = p->q_stride[1]; a.qss = p->q_stride[2];
    a.ksb = p->k_stride[0]; a.ksh = p->k_stride[1]; a.kss = p->k_stride[2];
    a.vsb = p->v_stride[0]; a.vsh = p->v_stride[1]; a.vss = p->v_stride[2];
    a.osb = p->o_stride[0]; a.osh = p->o_stride[1]; a.oss = p->o_stride[2];
    a.dosb = p->do_stride[0]; a.dosh = p->do_stride[1]; a.doss = p->do_stride[2];
    a.dqsb = p->dq_stride[0]; a.dqsh = p->dq_stride[1]; a.dqss = p->dq_stride[2];
    a.dksb = p->dk_stride[0]; a.dksh = p->dk_stride[1]; a.dkss = p->dk_stride[2];
    a.dvsb = p->dv_stride[0]; a.dvsh = p->dv_stride[1]; a.dvss = p->dv_stride[2];
    a.lsb = p->lse_stride[0]; a.lsh = p->lse_stride[1];
    a.B = p->B; a.H = p->H; a.S = p->S;
    a.scale = p->softmax_scale;
    a.scale2 = scale2_of(p->softmax_scale);
    a.negate = p->softmax_scale < 0.f;
    a.seed = p->seed;
    a.drop_thr = fa2_dropout_threshold(p->dropout_p);
    a.inv_keep = 1.f / (1.f - p->dropout_p);
    const bool causal = p->causal != 0, dropout = p->dropout_p > 0.f;
    a.drop_mask = dropout ? p->dropout_mask : nullptr;
    a.hgroup = 0;
    const hipStream_t st = (hipStream_t)stream;

    hipError_t e = hipSuccess;
    if (want_dq) {
        e = fa2::launch_bwd_dq(a, causal, dropout, st);  // also writes delta
        if (e != hipSuccess) return fail(FA2_ERR_LAUNCH, "dQ launch: %s", hipGetErrorString(e));
    } else if (want_delta) {
        e = fa2::launch_bwd_delta(a, st);
        if (e != hipSuccess) return fail(FA2_ERR_LAUNCH, "delta launch: %s", hipGetErrorString(e));
    }
    if (want_dkv) {
        e = fa2::launch_bwd_dkv(a, causal, dropout, st);
        if (e != hipSuccess) return fail(FA2_ERR_LAUNCH, "dK/dV launch: %s", hipGetErrorString(e));
    }
    return FA2_OK;
}

int fa2_bwd_f16(const fa2_bwd_params *p, int32_t mode, void *workspace, size_t workspace_bytes, void *stream) {
    g_err[0] = 0;
    int rc = bwd_precheck(p, mode);
    if (rc) return rc < 0 ? FA2_OK : rc;
    const size_t need = fa2_bwd_workspace_bytes(p->B, p->H, p->S);
    if (!workspace || workspace_bytes < need)
        return fail(FA2_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : 0);
    if (reinterpret_cast<uintptr_t>(workspace) & 15u)
        return fail(FA2_ERR_MISALIGNED, "workspace is not 16-byte aligned");
    return bwd_run(p, mode, workspace, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free backward: the workspace is `scratch`, a device array of
// FA2_BWD_SCRATCH_MAX_BYTES that every GPU the library runs on holds from the
// module's load until the process ends.  In host code `scratch` names a
// host-side stand-in, never the device memory: the device address comes from
// hipGetSymbolAddress, once per device with that device current, and only
// that address is passed on.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[FA2_BWD_SCRATCH_MAX_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's copy of `scratch` (set up on the
// first call on that device), or a status.
int scratch_for_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(FA2_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(FA2_ERR_LAUNCH, "device ordinal %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(FA2_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return FA2_OK;
}
}  // namespace

extern "C" {

size_t fa2_bwd_noalloc_scratch_bytes(int32_t B, int32_t H, int32_t S) {
    if (B <= 0 || H <= 0 || S <= 0) return 0;
    return delta_bytes(B, H, S) + terms_bytes(B, H, S);
}

int fa2_bwd_f16_noalloc(const fa2_bwd_params *p, int32_t mode, void *stream) {
    g_err[0] = 0;
    int rc = bwd_precheck(p, mode);
    if (rc) return rc < 0 ? FA2_OK : rc;
    const size_t need = fa2_bwd_noalloc_scratch_bytes(p->B, p->H, p->S);
    if (need > (size_t)FA2_BWD_SCRATCH_MAX_BYTES)
        return fail(FA2_ERR_WORKSPACE, "B=%d H=%d S=%d needs %zu bytes of scratch; fa2_bwd_f16_noalloc holds "
                    "%zu (FA2_BWD_SCRATCH_MAX_BYTES): use fa2_bwd_f16 with a workspace",
                    p->B, p->H, p->S, need, (size_t)FA2_BWD_SCRATCH_MAX_BYTES);
    void *ws = nullptr;
    if ((rc = scratch_for_current_device(&ws))) return rc;
    return bwd_run(p, mode, ws, stream);
}

int fa2_rope_f16(const fa2_rope_params *p, int32_t backward, void *stream) {
    g_err[0] = 0;
    if (!p) return fail(FA2_ERR_NULL_POINTER, "params is NULL");
    int rc = check_shape(p->B, p->H, p->S, p->D, 8);
    if (rc) return rc;
    if ((int64_t)p->B * p->H * p->S == 0) return FA2_OK;
    if ((rc = check_tensor("q", p->q, p->q_stride, p->B, p->H, p->S, false))) return rc;
    if ((rc = check_tensor("k", p->k, p->k_stride, p->B, p->H, p->S, false))) return rc;
    if ((rc = check_tensor("qo", p->qo, p->qo_stride, p->B, p->H, p->S, false))) return rc;
    if ((rc = check_tensor("ko", p->ko, p->ko_stride, p->B, p->H, p->S, false))) return rc;
    if (!p->cos || !p->sin) return fail(FA2_ERR_NULL_POINTER, "cos/sin is NULL");
    if ((reinterpret_cast<uintptr_t>(p->cos) | reinterpret_cast<uintptr_t>(p->sin)) & 3u)
        return fail(FA2_ERR_MISALIGNED, "cos/sin are not 4-byte aligned");
    if (p->cs_stride < 0 || p->sn_stride < 0) return fail(FA2_ERR_BAD_SHAPE, "negative cos/sin stride");
    fa2::RopeArgs a;
    a.q = static_cast<const _Float16 *>(p->q);
    a.k = static_cast<const _Float16 *>(p->k);
    a.qo = static_cast<_Float16 *>(p->qo);
    a.ko = static_cast<_Float16 *>(p->ko);
    a.cs = p->cos;
    a.sn = p->sin;
    a.qsb = p->q_stride[0]; a.qsh = p->q_stride[1]; a.qss = p->q_stride[2];
    a.ksb = p->k_stride[0]; a.ksh = p->k_stride[1]; a.kss = p->k_stride[2];
    a.oqb = p->qo_stride[0]; a.oqh = p->qo_stride[1]; a.oqs = p->qo_stride[2];
    a.okb = p->ko_stride[0]; a.okh = p->ko_stride[1]; a.oks = p->ko_stride[2];
    a.cs0 = p->cs_stride;
    a.sn0 = p->sn_stride;
    a.B = p->B; a.H = p->H; a.S = p->S;
    {
        const int64_t *st[4] = {p->q_stride, p->k_stride, p->qo_stride, p->ko_stride};
        int64_t half_strides = 0;   // fp16 strides: multiples of 8 keep 16-byte rows
        for (const int64_t *x : st) half_strides |= x[0] | x[1] | x[2];
        const uintptr_t ptrs = reinterpret_cast<uintptr_t>(p->q) | reinterpret_cast<uintptr_t>(p->k) |
                               reinterpret_cast<uintptr_t>(p->qo) | reinterpret_cast<uintptr_t>(p->ko) |
                               reinterpret_cast<uintptr_t>(p->cos) | reinterpret_cast<uintptr_t>(p->sin);
        a.vec16 = (ptrs & 15u) == 0 && (half_strides & 7) == 0 && ((p->cs_stride | p->sn_stride) & 3) == 0;
    }
    const hipError_t e = fa2::launch_rope(a, backward != 0, (hipStream_t)stream);
    if (e != hipSuccess) return fail(FA2_ERR_LAUNCH, "rope launch: %s", hipGetErrorString(e));
    return FA2_OK;
}

}  // extern "C"
