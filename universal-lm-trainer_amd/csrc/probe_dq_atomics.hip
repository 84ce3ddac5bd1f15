// probe_dq_atomics.hip -- measures what accumulating dQ with fp32 atomics would
// cost at benchmark configuration 2 (B*H = 96, S = 4096, D = 64, causal), the
// alternative to the split dQ pass (reference @ None:
// csrc/flash_attn_v100/flash_attn_v100_bwd.cu:433-506 runs a split pass too).
//
// A fused backward's workgroup owns a block of kb keys of one (b, h) and, for
// every 32-query tile at or below its diagonal, adds its 32 x 64 fp32 share of
// dQ into an accumulator.  Each kernel here issues exactly that traffic and
// nothing else (no matrix work): one workgroup per (key block, b*h), 4 waves,
// wave w adding rows 8w .. 8w+7 of each tile as 64-lane, 256-byte runs.
//   dq_atomic_f32<kb> : global_atomic_add_f32 (no return), the fused design
//   dq_store_f32<kb>  : plain stores of the same bytes, for comparison
// Without matrix work to hide behind, each kernel's duration is the floor the
// accumulation alone puts under a fused backward.  Run under rocprofv3
// --kernel-trace --stats, or alone (it prints its own HIP-event timings).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

constexpr int kHeads = 96, kS = 4096, kD = 64, kQT = 32;

template <int KB, bool ATOMIC>
__global__ __launch_bounds__(256) void dq_traffic(float *acc) {
    const int heads = kHeads;
    const int L = blockIdx.x;
    const int kblk = L / heads, bh = L - kblk * heads;     // a head's key blocks share an XCD
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *base = acc + (size_t)bh * kS * kD;
    const float val = 1.0f;
    for (int q0 = kblk * KB; q0 < kS; q0 += kQT) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            float *p = base + (size_t)(q0 + 8 * wave + r) * kD + lane;
            if (ATOMIC)
                __hip_atomic_fetch_add(p, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                *p = val;
        }
    }
}

#define CK(x)                                                                            \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess) {                                                          \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_));     \
            exit(1);                                                                     \
        }                                                                                \
    } while (0)

template <int KB, bool ATOMIC>
void run(float *acc, const char *name) {
    const int nblk = kS / KB;
    const dim3 grid(nblk * kHeads), block(256);
    // bytes one launch moves: 256 B per 64-lane run, 32 runs per tile
    double bytes = 0;
    for (int kb = 0; kb < nblk; ++kb) bytes += (double)(kS - kb * KB) / kQT * kQT * kD * 4;
    bytes *= kHeads;
    CK(hipMemset(acc, 0, (size_t)kHeads * kS * kD * 4));
    hipLaunchKernelGGL((dq_traffic<KB, ATOMIC>), grid, block, 0, 0, acc);   // warm-up
    CK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const int iters = 5;
    CK(hipEventRecord(e0));
    for (int i = 0; i < iters; ++i) hipLaunchKernelGGL((dq_traffic<KB, ATOMIC>), grid, block, 0, 0, acc);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, e0, e1));
    ms /= iters;
    printf("%-28s keys/workgroup %3d  %7.1f MB  %8.1f us  %6.2f TB/s\n", name, KB, bytes / 1e6, ms * 1e3,
           bytes / (ms * 1e-3) / 1e12);
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
}

}  // namespace

int main() {
    float *acc = nullptr;
    CK(hipMalloc(&acc, (size_t)kHeads * kS * kD * 4));
    run<128, true>(acc, "fp32 atomics (fused dQ)");
    run<256, true>(acc, "fp32 atomics (fused dQ)");
    run<128, false>(acc, "plain fp32 stores");
    run<256, false>(acc, "plain fp32 stores");
    CK(hipFree(acc));
    return 0;
}
