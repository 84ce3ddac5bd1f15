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
// HBM-bound: per (b, h, s) row, 128 bytes read and 128 written for q and for
// k; the cos/sin rows (256 bytes each) are shared by the H rows of a position
// and stay in cache.
//
// Vector path (16-byte aligned rows): eight lanes per row, lane j holding
// halves 8j .. 8j+7 of it in one 16-byte load; its rotation partner, halves
// 8j +- 32, sits in lane j ^ 4 of the same eight and arrives by a lane swap
// (no second read of the row).  Rows are numbered position-major with heads
// fastest, so a wave covers 8 heads of one position: the memory order of the
// fused-qkv layout train.py produces, and one cos/sin row for the whole wave.
// Scalar path (any even strides): one lane per pair of halves, as a fallback
// for rows that are only 4-byte aligned.
#include "fa2_device.h"
#include "fa2_kernels.h"

namespace fa2 {
namespace {

typedef float f8v __attribute__((ext_vector_type(8)));
// cos / sin rows are only guaranteed 16-byte alignment (the host's vector-path
// check), so their 8-float loads go through a type of that alignment.
typedef float f8v_a16 __attribute__((ext_vector_type(8), aligned(16)));

// One row of eight halves per lane: x = own halves, xp = partner halves,
// cs / snv = cos and the sine the formula multiplies (own index forward,
// partner index backward), sg = the sign of the partner term.
__device__ __forceinline__ h8 rope8(h8 x, h8 xp, f8v cs, f8v snv, float sg) {
#pragma clang fp contract(off)
    f8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float t = (float)x[e] * cs[e];
        const float u = (sg * (float)xp[e]) * snv[e];
        o[e] = t + u;
    }
    return __builtin_convertvector(o, h8);
}

__device__ __forceinline__ h8 swap4(h8 v) {   // the value held by lane ^ 4
    typedef int i4 __attribute__((ext_vector_type(4)));
    i4 w = __builtin_bit_cast(i4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __shfl_xor(w[i], 4);
    return __builtin_bit_cast(h8, w);
}

template <bool BACKWARD>
__global__ __launch_bounds__(256) void rope_vec_kernel(const RopeArgs a) {
    // B*H*S < 2^31 (host check): 32-bit row arithmetic
    const uint32_t H = (uint32_t)a.H, S = (uint32_t)a.S;
    const uint32_t rows = (uint32_t)a.B * S * H;
    const uint32_t r = blockIdx.x * 32u + (threadIdx.x >> 3);   // (b*S + s)*H + h
    if (r >= rows) return;                 // whole groups of 8 lanes leave together
    const int j = threadIdx.x & 7;         // halves 8j .. 8j+7
    const uint32_t bs = r / H;
    const int h = (int)(r - bs * H);
    const int b = (int)(bs / S), s = (int)(bs - (uint32_t)b * S);
    const float *csr = a.cs + (int64_t)s * a.cs0, *snr = a.sn + (int64_t)s * a.sn0;
    const f8v cs = *reinterpret_cast<const f8v_a16 *>(csr + 8 * j);
    // forward: sin at the own index, partner sign -1 for d < 32;
    // backward: sin at the partner index, partner sign +1 for d < 32.
    const f8v snv = *reinterpret_cast<const f8v_a16 *>(snr + 8 * (BACKWARD ? (j ^ 4) : j));
    const float sg = (j < 4) == BACKWARD ? 1.f : -1.f;
    const h8 xq = *reinterpret_cast<const h8 *>(a.q + b * a.qsb + h * a.qsh + s * a.qss + 8 * j);
    const h8 xk = *reinterpret_cast<const h8 *>(a.k + b * a.ksb + h * a.ksh + s * a.kss + 8 * j);
    const h8 pq = swap4(xq), pk = swap4(xk);
    *reinterpret_cast<h8 *>(a.qo + b * a.oqb + h * a.oqh + s * a.oqs + 8 * j) = rope8(xq, pq, cs, snv, sg);
    *reinterpret_cast<h8 *>(a.ko + b * a.okb + h * a.okh + s * a.oks + 8 * j) = rope8(xk, pk, cs, snv, sg);
}

template <bool BACKWARD>
__device__ __forceinline__ void rope_pair(const _Float16 *__restrict__ src, _Float16 *__restrict__ dst,
                                          const float *__restrict__ cs, const float *__restrict__ sn,
                                          int lane32) {
#pragma clang fp contract(off)
    const int d = 2 * lane32;
    const int dp = (lane32 < 16) ? d + 32 : d - 32;
    const h2 x = *reinterpret_cast<const h2 *>(src + d);
    const h2 xp = *reinterpret_cast<const h2 *>(src + dp);
    const int ds = BACKWARD ? dp : d;                                // index of the sine factor
    const float sg = (lane32 < 16) == BACKWARD ? 1.f : -1.f;
    const float t0 = (float)x[0] * cs[d];
    const float t1 = (float)x[1] * cs[d + 1];
    const float u0 = (sg * (float)xp[0]) * sn[ds];
    const float u1 = (sg * (float)xp[1]) * sn[ds + 1];
    h2 r;
    r[0] = (_Float16)(t0 + u0);
    r[1] = (_Float16)(t1 + u1);
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
    const bool vec = a.vec16;
    if (vec) {
        const uint32_t rows = (uint32_t)a.B * (uint32_t)a.S * (uint32_t)a.H;
        const dim3 grid((rows + 31u) / 32u), block(256);
        if (backward)
            hipLaunchKernelGGL(rope_vec_kernel<true>, grid, block, 0, st, a);
        else
            hipLaunchKernelGGL(rope_vec_kernel<false>, grid, block, 0, st, a);
    } else {
        const int nrb = (a.S + 7) / 8;
        const dim3 grid((unsigned)(nrb * a.B * a.H)), block(256);
        if (backward)
            hipLaunchKernelGGL(rope_kernel<true>, grid, block, 0, st, a);
        else
            hipLaunchKernelGGL(rope_kernel<false>, grid, block, 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace fa2
