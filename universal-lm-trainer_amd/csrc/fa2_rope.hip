// fa2_rope.hip -- fused rotary embedding on q and k for head_dim 64.
//
// Semantics (reference @ None: csrc/flash_attn_v100/fast_ops.cu:31-68):
//   forward : out[d] = x[d]*cos[d] + r[d]*sin[d],
//             r[d] = -x[d+32] (d < 32),  x[d-32] (d >= 32)
//   backward: gx[d]  = g[d]*cos[d] + sgn*g[dp]*sin[dp],
//             dp = d+32, sgn = +1 (d < 32);  dp = d-32, sgn = -1 (d >= 32)
// All in fp32 with separately rounded multiplies and add (no FMA
// contraction), one RNE rounding to fp16 -- bitwise equal to the eager fp32
// expression followed by .half().
//
// Mapping: one thread per (row, d pair), 32 threads per row; each thread
// handles the same (d, d+1) pair of the q row and of the k row.  HBM-bound:
// 2 x (read 128 B + write 128 B) per (b, h, s) row plus the cos/sin rows.
#include "fa2_device.h"
#include "fa2_kernels.h"

namespace fa2 {
namespace {

template <bool BACKWARD>
__device__ __forceinline__ void rope_pair(const _Float16 *__restrict__ src, _Float16 *__restrict__ dst,
                                          const float *__restrict__ cs, const float *__restrict__ sn,
                                          int lane32) {
#pragma clang fp contract(off)
    const int d = 2 * lane32;
    const int dp = (lane32 < 16) ? d + 32 : d - 32;
    const h2 x = *reinterpret_cast<const h2 *>(src + d);
    const h2 xp = *reinterpret_cast<const h2 *>(src + dp);
    float o0, o1;
    if (!BACKWARD) {
        const float sg = (lane32 < 16) ? -1.f : 1.f;
        const float t0 = (float)x[0] * cs[d];
        const float t1 = (float)x[1] * cs[d + 1];
        const float u0 = (sg * (float)xp[0]) * sn[d];
        const float u1 = (sg * (float)xp[1]) * sn[d + 1];
        o0 = t0 + u0;
        o1 = t1 + u1;
    } else {
        const float sg = (lane32 < 16) ? 1.f : -1.f;
        const float t0 = (float)x[0] * cs[d];
        const float t1 = (float)x[1] * cs[d + 1];
        const float u0 = (sg * (float)xp[0]) * sn[dp];
        const float u1 = (sg * (float)xp[1]) * sn[dp + 1];
        o0 = t0 + u0;
        o1 = t1 + u1;
    }
    h2 r;
    r[0] = (_Float16)o0;
    r[1] = (_Float16)o1;
    *reinterpret_cast<h2 *>(dst + d) = r;
}

template <bool BACKWARD>
__global__ __launch_bounds__(256) void rope_kernel(const RopeArgs a) {
    const int S = a.S;
    const int nrb = (S + 7) / 8;
    const int bh = blockIdx.x / nrb;
    const int s = (blockIdx.x - bh * nrb) * 8 + (threadIdx.x >> 5);
    if (s >= S) return;
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane32 = threadIdx.x & 31;
    const float *cs = a.cs + s * a.cs0;
    const float *sn = a.sn + s * a.sn0;
    rope_pair<BACKWARD>(a.q + b * a.qsb + h * a.qsh + s * a.qss, a.qo + b * a.oqb + h * a.oqh + s * a.oqs, cs, sn,
                        lane32);
    rope_pair<BACKWARD>(a.k + b * a.ksb + h * a.ksh + s * a.kss, a.ko + b * a.okb + h * a.okh + s * a.oks, cs, sn,
                        lane32);
}

}  // namespace

hipError_t launch_rope(const RopeArgs &a, bool backward, hipStream_t st) {
    const int nrb = (a.S + 7) / 8;
    const dim3 grid((unsigned)(nrb * a.B * a.H)), block(256);
    if (backward)
        hipLaunchKernelGGL(rope_kernel<true>, grid, block, 0, st, a);
    else
        hipLaunchKernelGGL(rope_kernel<false>, grid, block, 0, st, a);
    return hipGetLastError();
}

}  // namespace fa2
