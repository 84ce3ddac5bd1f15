// ref_hash_harness.hip -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
//
// Runs the reference's own dropout hash on the GPU so that the oracle's
// restatement can be compared with it bit for bit.  The reference functions
// `hash_u32` and `dropout_keep` (reference @ None:
// csrc/flash_attn_v100/fa_common.cuh:21-38) are compiled from the reference's
// source lines themselves: oracle/build_ref.py copies exactly those lines into
// a temporary file outside the repository and passes its path as
// FA2REF_HASH_LINES.  They need no header (plain integer code under
// __device__ __forceinline__, which hipcc accepts as written); the rest of
// fa_common.cuh includes <cuda_fp16.h>, which this image does not have.
//
// Exports (host arrays in, host arrays out; the harness allocates and frees
// its own device buffers, returns the HIP error code):
//   fa2ref_dropout_keep(seed, row, col, bh, p, keep, n)
//   fa2ref_hash_u32(x, out, n)
#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef FA2REF_HASH_LINES
#error "FA2REF_HASH_LINES must name the extracted reference lines (oracle/build_ref.py)"
#endif

namespace fav100 {
#include FA2REF_HASH_LINES
}  // namespace fav100

namespace {

__global__ void keep_kernel(const uint32_t *seed, const int32_t *row, const int32_t *col, const uint32_t *bh,
                            const float *p, uint8_t *keep, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) keep[i] = fav100::dropout_keep(seed[i], row[i], col[i], bh[i], p[i]) ? 1 : 0;
}

__global__ void hash_kernel(const uint32_t *x, uint32_t *out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = fav100::hash_u32(x[i]);
}

struct Buffers {
    void *p[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    ~Buffers() {
        for (void *q : p)
            if (q) (void)hipFree(q);
    }
};

#define FA2REF_TRY(x)                      \
    do {                                   \
        const hipError_t e_ = (x);         \
        if (e_ != hipSuccess) return (int)e_; \
    } while (0)

}  // namespace

extern "C" int fa2ref_dropout_keep(const uint32_t *seed, const int32_t *row, const int32_t *col, const uint32_t *bh,
                                   const float *p, uint8_t *keep, int64_t n) {
    if (n <= 0) return 0;
    Buffers b;
    const size_t w = (size_t)n * 4;
    for (int i = 0; i < 5; ++i) FA2REF_TRY(hipMalloc(&b.p[i], w));
    FA2REF_TRY(hipMalloc(&b.p[5], (size_t)n));
    FA2REF_TRY(hipMemcpy(b.p[0], seed, w, hipMemcpyHostToDevice));
    FA2REF_TRY(hipMemcpy(b.p[1], row, w, hipMemcpyHostToDevice));
    FA2REF_TRY(hipMemcpy(b.p[2], col, w, hipMemcpyHostToDevice));
    FA2REF_TRY(hipMemcpy(b.p[3], bh, w, hipMemcpyHostToDevice));
    FA2REF_TRY(hipMemcpy(b.p[4], p, w, hipMemcpyHostToDevice));
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(keep_kernel, dim3((unsigned)blocks), dim3(256), 0, 0, (const uint32_t *)b.p[0],
                       (const int32_t *)b.p[1], (const int32_t *)b.p[2], (const uint32_t *)b.p[3],
                       (const float *)b.p[4], (uint8_t *)b.p[5], n);
    FA2REF_TRY(hipGetLastError());
    FA2REF_TRY(hipMemcpy(keep, b.p[5], (size_t)n, hipMemcpyDeviceToHost));
    return 0;
}

extern "C" int fa2ref_hash_u32(const uint32_t *x, uint32_t *out, int64_t n) {
    if (n <= 0) return 0;
    Buffers b;
    const size_t w = (size_t)n * 4;
    FA2REF_TRY(hipMalloc(&b.p[0], w));
    FA2REF_TRY(hipMalloc(&b.p[1], w));
    FA2REF_TRY(hipMemcpy(b.p[0], x, w, hipMemcpyHostToDevice));
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(hash_kernel, dim3((unsigned)blocks), dim3(256), 0, 0, (const uint32_t *)b.p[0],
                       (uint32_t *)b.p[1], n);
    FA2REF_TRY(hipGetLastError());
    FA2REF_TRY(hipMemcpy(out, b.p[1], w, hipMemcpyDeviceToHost));
    return 0;
}
