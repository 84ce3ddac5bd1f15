// fa2_kernels.h -- kernel argument blocks and launch entry points shared by
// the C ABI layer (fa2_capi.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa2 {

// All strides are in elements.  Kernel-side invariants established by the
// host (fa2_capi.hip): D == 64, base pointers 16-byte aligned, (b,h,s)
// strides multiples of 8, scale2 > 0 and finite.
struct FwdArgs {
    const _Float16 *q, *k, *v;
    _Float16 *o;
    float *lse;
    int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss, osb, osh, oss, lsb, lsh;
    int B, H, S;         // S: query rows (q, o, lse)
    int Sk;              // key / value rows
    int coff;            // causal: key j visible to query i iff j <= i + coff
    // Split forward (launch_fwd_split): nsplit slices of split_keys keys (a
    // multiple of 64); partials [nsplit, B*H, S] x (64 fp32 O) and x (max, sum).
    int nsplit;
    int split_keys;
    float *part_o;
    float *part_ml;
    float scale2;        // |softmax_scale| * log2(e), at least FLT_MIN
    int negate;          // softmax_scale < 0: the Q operand is negated
    uint32_t seed;       // dropout hash seed
    uint32_t drop_thr;   // keep iff (hash >> 8) >= drop_thr
    float inv_keep;      // 1 / (1 - p)
    // Dropout keep bits (dmask_word layout) written for the backward, or null.
    uint32_t *drop_mask;
    // Workgroup order (query_block_order): heads per group, 0 = plain order.
    int hgroup;
};

struct BwdArgs {
    const _Float16 *q, *k, *v, *o, *dout;
    const float *lse;
    _Float16 *dq, *dk, *dv;
    float *delta;        // [B*H, S] fp32 workspace: delta = rowsum(dO * O)
    float *lse2;         // [B*H, S] fp32 workspace: LSE * log2(e), right after delta
    // Per 32-query block of each (b,h) (blocks of 256 bytes, S rounded up to
    // 32): the block's 32 values of -LSE*log2(e)/scale2, then its 32 values of
    // -delta, fp32 -- the per-row terms the dK/dV pass starts its S and dP
    // accumulators from.
    float *rowterm;
    int64_t qsb, qsh, qss, ksb, ksh, kss, vsb, vsh, vss;
    int64_t osb, osh, oss, dosb, dosh, doss;
    int64_t dqsb, dqsh, dqss, dksb, dksh, dkss, dvsb, dvsh, dvss;
    int64_t lsb, lsh;
    int B, H, S;
    float scale;         // signed softmax scale (multiplies dQ and dK)
    float scale2;        // |softmax_scale| * log2(e), at least FLT_MIN
    int negate;          // softmax_scale < 0: the K operand of S is negated
    uint32_t seed;
    uint32_t drop_thr;
    float inv_keep;
    // Dropout keep bits the forward wrote (dmask_word layout), or null: the
    // passes then evaluate the hash themselves.
    const uint32_t *drop_mask;
    // dK/dV pass: one workgroup runs key blocks j and nkb - 1 - j (causal).
    bool dkv_pair;
    // dQ pass workgroup order (query_block_order): heads per group, 0 = plain.
    int hgroup;
};

struct RopeArgs {
    const _Float16 *q, *k;
    _Float16 *qo, *ko;
    const float *cs, *sn;
    int64_t qsb, qsh, qss, ksb, ksh, kss, oqb, oqh, oqs, okb, okh, oks;
    int64_t cs0, sn0;
    int B, H, S;
    // Every row pointer (q, k, qo, ko, cos, sin bases and strides) 16-byte
    // aligned: the vector kernel; otherwise the 4-byte one.
    bool vec16;
};

// Compute units of the current device (cached per device; 256 on MI355X).
// Launchers use it to size grids against the slots of two workgroups per CU.
int device_cus();

// Launchers; each returns the hipError_t of its launch.
hipError_t launch_fwd(const FwdArgs &a, bool causal, bool dropout, hipStream_t st);
// The forward over a.nsplit key slices (partials into a.part_o / a.part_ml), then their merge.
hipError_t launch_fwd_split(const FwdArgs &a, bool causal, bool dropout, hipStream_t st);
// One query (S = 1), no dropout: the VALU decode kernel over a.nsplit slices
// (a.part_o null when nsplit = 1), then the merge when nsplit > 1.
hipError_t launch_fwd_decode(const FwdArgs &a, bool causal, hipStream_t st);
hipError_t launch_bwd_delta(const BwdArgs &a, hipStream_t st);
hipError_t launch_bwd_dq(const BwdArgs &a, bool causal, bool dropout, hipStream_t st);
hipError_t launch_bwd_dkv(const BwdArgs &a, bool causal, bool dropout, hipStream_t st);
hipError_t launch_rope(const RopeArgs &a, bool backward, hipStream_t st);

}  // namespace fa2
