// fa2_device.h -- device-side building blocks shared by the gfx950 attention
// kernels: vector types, the fp16 MFMA wrapper, LDS tile swizzles and
// transposing reads, direct global->LDS transfers, the dropout hash and small
// cross-lane helpers.
//
// Register layouts of v_mfma_f32_32x32x16_f16 (wave64, lane = 32*g2 + c):
//   A operand (32 x 16, half8): lane holds A[m = c][k = 8*g2 + e], e = 0..7
//   B operand (16 x 32, half8): lane holds B[k = 8*g2 + e][n = c]
//   C/D       (32 x 32, 16 f32): register r = 4*i + j holds
//             D[m = 8*i + 4*g2 + j][n = c]
// The product only needs A and B to agree on which logical k sits in
// (g2, e), so the kernels feed a logical k order of their own choosing into
// both operands.  The one they use lets an accumulator be reused as the B
// operand of the next MFMA without leaving registers: registers 8*hh .. 8*hh+7
// of an accumulator hold rows 16*hh + 8*(e/4) + 4*g2 + (e%4), which is exactly
// the k order of a 16-deep B operand.  The A operand read from LDS must then
// present its k index in that order, which the transposing LDS reads below
// (ds_read_b64_tr_b16) deliver directly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa2 {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

constexpr int HD = 64;        // head dimension (the only one supported)
constexpr int LDR = HD + 8;   // LDS row stride in halves: 144 B keeps 16-byte
                              // reads by 16 lanes on distinct banks
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

__device__ __forceinline__ f16x mfma32(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Placed first in the body of a rarely taken, wave-uniform branch (causal
// diagonal masking, lazy rescale): a volatile asm statement cannot be
// speculated, so the compiler keeps a real branch instead of if-converting the
// body into selects that would then run on every tile.
#define FA2_COLD_BRANCH() asm volatile("" ::: "memory")

// Kernel-local lambdas are always inlined: an out-of-line call would pass the
// register arrays they work on through scratch memory.
#define FA2_INLINE __attribute__((always_inline))

// First MFMA of an accumulation chain: C is the constant zero.
__device__ __forceinline__ f16x mfma32_first(h8 a, h8 b) {
    const f16x z = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ f16x zero16() {
    f16x z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

__device__ __forceinline__ h8 zero_h8() {
    h8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (_Float16)0.f;
    return z;
}

// Transposing operand read (ds_read_b64_tr_b16).  From a row-major LDS tile
// M[k][n] (row stride LD halves), lane 32*g2 + c receives
//     M[k0 + 8*a + 4*g2 + j][n0 + c]   in slot e = 4*a + j  (a = 0..1, j = 0..3),
// i.e. the A or B operand of a 16-deep MFMA step whose lane index runs along
// n and whose k order is the accumulator-chaining order above -- without a
// transposed copy of the tile.
// Instruction semantics (measured on gfx950 with an in-bounds probe): within
// each group of 16 lanes, lane i receives element (i & 3) of the 8-byte
// segments addressed by lanes 4*e + (i >> 2), e = 0..3.  So source lane s of
// group G points at row k0 + 8a + 4*(G>>1) + (s>>2), column n0 + 16*(G&1) +
// 4*(s&3), and two reads (a = 0, 1) fill the 8 slots.  Rows must be 8-byte
// aligned (LD and n0 multiples of 4).
typedef short s4v __attribute__((ext_vector_type(4)));
typedef short s8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s4v lds_s4v;

template <int LD>
__device__ __forceinline__ h8 tr_read8(const _Float16 *tile, int k0, int n0) {
    const int L = threadIdx.x & 63;
    const int G = L >> 4, s = L & 15;
    const int row = k0 + 4 * (G >> 1) + (s >> 2);
    const int col = n0 + 16 * (G & 1) + 4 * (s & 3);
    const __attribute__((address_space(3))) _Float16 *t =
        (const __attribute__((address_space(3))) _Float16 *)tile;
    const s4v r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v *)(t + row * LD + col));
    const s4v r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v *)(t + (row + 8) * LD + col));
    const s8v both = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(h8, both);
}

// ---------------------------------------------------------------------------
// Swizzled 64 x 64 fp16 tiles for direct global->LDS loads.
//
// A tile is 512 chunks of 16 bytes (8 halves); logical chunk ch (0..7) of row
// r sits at chunk position 8*r + (ch ^ f(r)).  The XOR pattern is chosen per
// read pattern so that the reads of one LDS pass touch distinct banks (for 32
// and for 64 four-byte banks):
//   * swz_rows(r): 16-byte reads of consecutive rows at one logical chunk
//     (MFMA operands whose lane index runs along the rows);
//   * swz_tr(r)  : transposing 8-byte reads of 4 rows x 32 bytes per 16 lanes
//     (ds_read_b64_tr_b16 operands).
// All depend on r & 15 only, so rows 16 apart differ by a constant offset.
//   * swz_both(r): both of the above on the same tile (an operand read as
//     rows by one MFMA and transposed by another).
__device__ __forceinline__ int swz_rows(int r) { return (r ^ ((r >> 3) & 1)) & 7; }
__device__ __forceinline__ int swz_tr(int r) { return ((2 * r) & 6) | ((r >> 2) & 1); }
__device__ __forceinline__ int swz_both(int r) { return swz_tr(r) ^ (((r >> 3) & 1) << 1); }

typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte global->LDS transfer per lane (global_load_lds_dwordx4): lane L
// of the wave writes the 16 bytes at byte address base + off to LDS bytes
// [dst + 16*L, +16).  `base` (a wave-uniform 64-bit address held in SGPRs)
// and `dst` must be wave-uniform; `off` is the lane's 32-bit byte offset, so
// a tile's per-lane offsets stay in registers while only the scalar base
// moves from tile to tile.  Completion is tracked by vmcnt only, so the
// reader waits with vm_wait<N>() and a workgroup barrier (lds_barrier()).
// Written as inline assembly: the compiler cannot tell which LDS reads a
// transfer may feed and would otherwise put a vmcnt(0) -- a full drain of the
// prefetch pipeline -- in front of them.  M0 (the LDS base of the transfer)
// is saved and restored around it, since the compiler reserves that register.
__device__ __forceinline__ void lds_dma16(const void *base, uint32_t off, void *dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)dst);
    // (readfirstlane returns int: each half goes through uint32_t so that the
    // low word is zero-extended, not sign-extended, into the 64-bit address.)
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(sb), "s"(lds));
}

// s * v for s, v < 2^24 with the product below 2^32 (v_mul_u32_u24, a
// full-rate instruction; s wave-uniform).  Written as assembly: from the
// same product in C the compiler forms v_mad_u64_u32, a quarter-rate
// instruction, which in per-tile address arithmetic costs more than the
// rest of that arithmetic together.
__device__ __forceinline__ uint32_t mul_u24(uint32_t s, uint32_t v) {
    uint32_t r;
    asm("v_mul_u32_u24 %0, %1, %2" : "=v"(r) : "s"(s), "v"(v));
    return r;
}

// LDS byte address of a __shared__ object, for the forms below that take the
// destination as an integer (converted once, outside the tile loop, instead
// of a generic-to-LDS pointer conversion at every transfer).
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const lds_void *)p;
}

// lds_dma16 / lds_dma4 with a wave-uniform 64-bit byte address and an LDS
// byte address, both already scalar (no conversion or readfirstlane).
__device__ __forceinline__ void lds_dma16_at(uint64_t base, uint32_t off, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds));
}
__device__ __forceinline__ void lds_dma4_at(uint64_t base, uint32_t off, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "global_load_lds_dword %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds));
}

// The 4-byte form (global_load_lds_dword): lane L writes 4 bytes to LDS
// bytes [dst + 4*L, +4).
__device__ __forceinline__ void lds_dma4(const void *base, uint32_t off, void *dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)dst);
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "global_load_lds_dword %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(sb), "s"(lds));
}

// Wait until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the release fence of __syncthreads(), whose
// vmcnt(0) would also drain every prefetch still in flight.  Outstanding LDS
// reads are drained first; global->LDS transfers are waited for explicitly
// with vm_wait.  The "memory" clobber keeps the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Transposing operand read from a swz_tr-swizzled 64-row tile: the result of
// tr_read8<64>(tile, k0, n0) for the unswizzled tile.  `lane_off` (bytes) is
// tr_lane_off(n0) for this lane; k0 must be a multiple of 8.
__device__ __forceinline__ int tr_lane_off(int n0) {
    const int L = threadIdx.x & 63;
    const int G = L >> 4, s = L & 15;
    const int row = 4 * (G >> 1) + (s >> 2);               // row within an 8-row group
    const int col = n0 + 16 * (G & 1) + 4 * (s & 3);
    return row * 128 + (((col >> 3) ^ swz_tr(row)) << 4) + 2 * (col & 7);
}

__device__ __forceinline__ h8 tr_read8_sw(const _Float16 *tile, int lane_off, int k0) {
    const char *base = reinterpret_cast<const char *>(tile) + lane_off + k0 * 128;
    const __attribute__((address_space(3))) char *t = (const __attribute__((address_space(3))) char *)base;
    const s4v r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v *)(t));
    const s4v r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v *)(t + 8 * 128));
    const s8v both = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(h8, both);
}

// The same read from a swz_both-swizzled tile.  Its swizzle also depends on
// row bit 3, so the two 8-row halves of a 16-row step have their own lane
// offsets: tr_both_off(n0, 0) for rows k0 .. k0+7, tr_both_off(n0, 1) for
// rows k0+8 .. k0+15; k0 must be a multiple of 16.
__device__ __forceinline__ int tr_both_off(int n0, int hi) {
    const int L = threadIdx.x & 63;
    const int G = L >> 4, s = L & 15;
    const int row = 4 * (G >> 1) + (s >> 2) + 8 * hi;      // row within a 16-row group
    const int col = n0 + 16 * (G & 1) + 4 * (s & 3);
    return row * 128 + (((col >> 3) ^ swz_both(row)) << 4) + 2 * (col & 7);
}

__device__ __forceinline__ h8 tr_read8_both(const _Float16 *tile, int off_lo, int off_hi, int k0) {
    const char *base = reinterpret_cast<const char *>(tile) + k0 * 128;
    const __attribute__((address_space(3))) char *t = (const __attribute__((address_space(3))) char *)base;
    const s4v r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v *)(t + off_lo));
    const s4v r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v *)(t + off_hi));
    const s8v both = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(h8, both);
}

// Registers 8*hh .. 8*hh+7 of an accumulator, rounded to fp16 (RNE): the B
// operand of the next 16-deep MFMA step.
__device__ __forceinline__ h8 acc_to_h8(const f16x &acc, int hh) {
    f8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = acc[8 * hh + e];
    return __builtin_convertvector(x, h8);
}

// Flips the sign of all eight halves when `neg` (exact), used to fold a
// negative softmax scale into one operand: one xor per register with both
// halves' sign bits, where the fp16 negation and a select took four
// instructions per register.
__device__ __forceinline__ h8 neg_h8_if(h8 v, bool neg) {
    typedef uint32_t u4w __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(h8, __builtin_bit_cast(u4w, v) ^ (neg ? 0x80008000u : 0u));
}

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

// Stores a wave's 32 x 64 output block held as two 32x32 MFMA accumulators
// (acc0: columns 0..31, acc1: 32..63 of each row; lane (c, g2) holds row c,
// columns 32*db + 8i + 4*g2 + j in element 4i + j), scaled by `mul`, as fp16
// rows dst + r * stride for r < nrows.  Direct stores would touch 32 rows per
// instruction in 8-byte pieces; the block goes through `blk`, a 4 KB
// wave-private LDS slice no other wave touches meanwhile (row r, 16-byte
// chunk ch at chunk ch ^ (r & 7): the row reads are conflict-free, the
// 8-byte writes put rows 8 apart on the same banks), and leaves as
// whole 128-byte rows, 8 lanes x 16 bytes (8-byte halves unless `vec16`:
// dst and stride multiples of 8 elements).
__device__ __forceinline__ void store_rows_f16(const f16x &acc0, const f16x &acc1, float mul, char *blk,
                                               _Float16 *dst, int64_t stride, int nrows, bool vec16) {
    const int lane = threadIdx.x & 63, c = lane & 31, g2 = lane >> 5;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f4 x;
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = (db ? acc1 : acc0)[4 * i + j] * mul;
            *reinterpret_cast<h4 *>(blk + c * 128 + (((4 * db + i) ^ (c & 7)) << 4) + 8 * g2) =
                __builtin_convertvector(x, h4);
        }
    const int ch = lane & 7;   // lane: chunk ch of rows 8k + (lane >> 3)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int r = 8 * k + (lane >> 3);
        const h8 v = *reinterpret_cast<const h8 *>(blk + r * 128 + ((ch ^ (r & 7)) << 4));
        if (r < nrows) {
            _Float16 *p = dst + r * stride + 8 * ch;
            if (vec16) {
                *reinterpret_cast<h8 *>(p) = v;
            } else {
                *reinterpret_cast<h4 *>(p) = __builtin_shufflevector(v, v, 0, 1, 2, 3);
                *reinterpret_cast<h4 *>(p + 4) = __builtin_shufflevector(v, v, 4, 5, 6, 7);
            }
        }
    }
}

// acc + sum of the eight halves, two per v_dot2_f32_f16 (fp32 accumulation).
__device__ __forceinline__ float sum_h8(h8 v, float acc) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2 pr;
        pr[0] = v[2 * i];
        pr[1] = v[2 * i + 1];
        acc = __builtin_amdgcn_fdot2(pr, one, acc, false);
    }
    return acc;
}

// Dropout keep decision for element (row = query, col = key) of head bh.
// The integer function is the reference's (reference @ None:
// csrc/flash_attn_v100/fa_common.cuh:21-38): the "lowbias32" finaliser over
// seed*0x9E3779B1 ^ (row+1)*0x85EBCA6B ^ (col+1)*0xC2B2AE35 ^ (bh+1)*0x27D4EB2F,
// keep iff (h >> 8) * 2^-24 >= p.  Since (h >> 8) < 2^24 that fp32 compare is
// exact and equals (h >> 8) >= thr with thr = ceil(p * 2^24), computed on the
// host, so the kernels stay in integer arithmetic.  p < 1 gives thr < 2^24,
// so (h >> 8) >= thr is h >= thr * 2^8, a compare against a loop-invariant
// bound with no shift per element.
// The hash input is (seed and head terms) ^ row term ^ column term.  A lane
// that keeps one query (or one key) over many elements computes that part once
// (dropout_row_part / dropout_col_part) and adds the other term per element.
__device__ __forceinline__ uint32_t dropout_row_term(int row) { return (uint32_t)(row + 1) * 0x85EBCA6Bu; }
__device__ __forceinline__ uint32_t dropout_col_term(int col) { return (uint32_t)(col + 1) * 0xC2B2AE35u; }
__device__ __forceinline__ uint32_t dropout_row_part(uint32_t seed, int row, uint32_t bh) {
    return (seed * 0x9E3779B1u) ^ dropout_row_term(row) ^ ((bh + 1u) * 0x27D4EB2Fu);
}
__device__ __forceinline__ uint32_t dropout_col_part(uint32_t seed, int col, uint32_t bh) {
    return (seed * 0x9E3779B1u) ^ dropout_col_term(col) ^ ((bh + 1u) * 0x27D4EB2Fu);
}
// The finaliser (lowbias32) of the full hash input x.
__device__ __forceinline__ uint32_t dropout_mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}
// The finaliser split for callers that share the column part between lanes.
// Its first step distributes over the xor of the two parts:
//   x ^ (x >> 16) = (r ^ (r >> 16)) ^ (k ^ (k >> 16))   for x = r ^ k,
// so dropout_xs16 of the row part and of the column term can be formed apart.
// Its last step folds into the keep compare: with T = thr << 8 and x4 the
// value before x4 ^ (x4 >> 16),
//   x4 ^ (x4 >> 16) >= T   <=>   (x4 ^ (T >> 16)) >= T,
// since both sides have the high half of x4 and, where that equals T's high
// half, the same low half.  dropout_mix_tail returns x4 ^ (T >> 16).
__device__ __forceinline__ uint32_t dropout_xs16(uint32_t v) { return v ^ (v >> 16); }
__device__ __forceinline__ uint32_t dropout_mix_tail(uint32_t x1, uint32_t thi) {
    x1 *= 0x7feb352du;
    x1 ^= x1 >> 15;
    x1 *= 0x846ca68bu;
    return x1 ^ thi;
}
// Keep decision from the full hash input x.
__device__ __forceinline__ bool dropout_keep_hashed(uint32_t x, uint32_t thr) {
    return dropout_mix(x) >= (thr << 8);
}
__device__ __forceinline__ bool dropout_keep(uint32_t seed, int row, int col, uint32_t bh,
                                             uint32_t thr) {
    return dropout_keep_hashed(dropout_row_part(seed, row, bh) ^ dropout_col_term(col), thr);
}

// 1/(1-p) if bit `bit` of the keep word w is set, else 0: the bit sign-
// extended (v_bfe_i32: 0 or all ones) masks the multiplier's bits, with no
// compare.
__device__ __forceinline__ float keep_multiplier(uint32_t w, int bit, float inv_keep) {
    const uint32_t sel = (uint32_t)__builtin_amdgcn_sbfe((int)w, bit, 1);
    return __builtin_bit_cast(float, sel & __builtin_bit_cast(uint32_t, inv_keep));
}

// Dropout keep bits, written by the forward and read by both backward passes
// instead of evaluating the hash again.  One 32-bit word per (b*H + h,
// 64-key tile t64, half g2, query q) at word index dmask_word(...): keys in
// tiles of 64 with dmask_tiles(S) = 2 * ceil(S / 128) tiles (the dK/dV pass
// reads both 64-key tiles of its 128-key block), queries padded to
// dmask_rows(S) = R = S rounded up to 256 (whole query blocks of every pass).
// Without the causal mask a run of R words per (tile, half); with it, tile
// t64 keeps only queries from rb = 128 * (t64 / 2) on -- the first query of
// its 128-key block, from where the dK/dV pass reads; every earlier query
// sees none of its keys -- in runs of R - rb words: about half the bytes.
// Bit 31 - (16*kb + 8*hh + e) of word g2 is key 64*t64 + 32*kb + 16*hh +
// 8*(e>>2) + 4*g2 + (e&3): the forward's own register order, shifted into
// the word element by element, so each lane builds one word per tile.
__device__ __forceinline__ int dmask_tiles(int S) { return 2 * ((S + 127) / 128); }
__device__ __forceinline__ int dmask_rows(int S) { return (S + 255) & ~255; }
// Words of one (tile, half) run: queries dmask_row0 .. R-1.
__device__ __forceinline__ int dmask_row0(bool causal, int t64) { return causal ? 128 * (t64 >> 1) : 0; }
__device__ __forceinline__ int dmask_run(bool causal, int S, int t64) { return dmask_rows(S) - dmask_row0(causal, t64); }
__device__ __forceinline__ int64_t dmask_word(bool causal, int bh, int S, int t64, int g2, int q) {
    const int64_t R = dmask_rows(S);
    if (!causal) return ((int64_t)bh * dmask_tiles(S) + t64) * 2 * R + (int64_t)g2 * R + q;
    // Blocks j < t64 / 2 hold 4 runs each of R - 128 j words.
    const int64_t J = dmask_tiles(S) >> 1, j = t64 >> 1, n = R - 128 * j;
    const int64_t head = 4 * J * R - 256 * J * (J - 1), before = 4 * j * R - 256 * j * (j - 1);
    return (int64_t)bh * head + before + (int64_t)(t64 & 1) * 2 * n + (int64_t)g2 * n + (q - 128 * j);
}

// Workgroup order of the query-block kernels (forward, dQ pass): workgroup L
// of a grid of nq * BH -> its query slot (0 = the head's last, heaviest
// query block) and its head bh.  Workgroups go to the 8 XCDs in turn
// (L % 8), each XCD with its own L2.
//   * G = 0: query slots outermost, heads fastest.  With BH a multiple of 8
//     a head's workgroups share one XCD, heaviest first over the whole grid,
//     but BH workgroups apart in time.
//   * G > 0 (the host passes it only when BH is a multiple of 8): XCD x takes
//     the heads x + 8 y and runs them in groups of G heads, query slots
//     heaviest first within each group, so that the query blocks of a head
//     run at about the same time and share its K / V tiles in the XCD's L2.
__device__ __forceinline__ void query_block_order(int L, int BH, int nq, int G, int &qslot, int &bh) {
    if (G > 0) {
        const int xcd = L & 7, i = L >> 3;
        const int per = G * nq;                       // workgroups of a full group
        const int grp = i / per, r = i - grp * per;
        const int gsz = min(G, (BH >> 3) - grp * G);  // the last group may be smaller
        qslot = r / gsz;
        bh = 8 * (grp * G + r - qslot * gsz) + xcd;
    } else {
        qslot = L / BH;
        bh = L - qslot * BH;
    }
}

}  // namespace fa2
