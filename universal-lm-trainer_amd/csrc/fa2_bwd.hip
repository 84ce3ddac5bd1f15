// fa2_bwd.hip -- causal FlashAttention-2 backward for gfx950 (MI355X).
//
// With S2 = scale*log2(e) * q.k and lse in natural log (the reference's
// formulas, reference @ None: csrc/flash_attn_v100/flash_attn_v100_bwd.cu:10-25):
//   P     = exp2(S2 - lse*log2(e))           (recomputed, never stored)
//   P_d   = keep * P / (1-p)                 (same hash as the forward)
//   delta = rowsum(O * dO)
//   dS    = P_d * dP - P * delta,  dP = dO V^T
//   dV    = P_d^T dO,  dK = scale * dS^T Q,  dQ = scale * dS K
//
// dQ accumulation: split pass, like the reference (its dQ and dK/dV kernels,
// bwd.cu:66-428), with no atomics:
//   * bwd_dq_pipe_kernel: a workgroup owns 256 queries (128 for S <= 1024),
//     keeps Q^T, dO^T, lse and delta of its queries in registers and streams
//     key tiles (K, V row-major via LDS; K^T operands come from transposing
//     ds_read_b64_tr_b16 reads) in order.  It also computes delta itself (the
//     reference's pre-pass, bwd.cu:42-61) from the O and dO rows it holds and
//     stores it, with the row terms, for the dK/dV pass.  S^T and dP^T accumulators give each lane one query, so
//     lse/delta are per-lane scalars and dS^T feeds the dQ^T = K^T dS^T MFMA
//     straight from registers.
//   * bwd_dkv_pipe_kernel: a workgroup owns 128 keys (32 per wave, K^T and
//     V^T in registers), streams query tiles (Q, dO row-major, lse, delta via
//     LDS; Q^T and dO^T operands through transposing reads) and accumulates
//     dK^T and dV^T in registers; P and dS feed the dV/dK MFMAs straight from
//     the S/dP accumulators.
#include "fa2_device.h"
#include "fa2_kernels.h"

namespace fa2 {
namespace {

// Word index of query q's term `which` (0: -LSE*log2(e)/scale2, 1: -delta),
// fp32, in the workspace's per-row terms: blocks of 64 words per 32 queries of
// a (b,h), the 32 first terms then the 32 second terms -- one 32-query tile's
// block is one 256-byte transfer.
__device__ __forceinline__ int64_t row_term_word(int S, int bh, int q, int which) {
    const int nb = (S + 31) >> 5;
    return ((int64_t)bh * nb + (q >> 5)) * 64 + which * 32 + (q & 31);
}
// Writes both terms of query q (lse2 = LSE * log2(e)).
__device__ __forceinline__ void store_row_terms(const BwdArgs &a, int bh, int q, float lse2, float delta) {
    a.rowterm[row_term_word(a.S, bh, q, 0)] = -lse2 / a.scale2;
    a.rowterm[row_term_word(a.S, bh, q, 1)] = -delta;
}

// ---------------------------------------------------------------------------
// delta only (used when the caller asks for delta without dQ): 8 lanes/row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bwd_delta_kernel(const BwdArgs a) {
    const int S = a.S;
    const int nrb = (S + 31) / 32;
    const int bh = blockIdx.x / nrb;
    const int row = (blockIdx.x - bh * nrb) * 32 + (threadIdx.x >> 3);
    const int b = bh / a.H, h = bh - b * a.H;
    const int part = threadIdx.x & 7;
    float sum = 0.f;
    if (row < S) {
        const h8 ov = *reinterpret_cast<const h8 *>(a.o + b * a.osb + h * a.osh + row * a.oss + 8 * part);
        const h8 dv = *reinterpret_cast<const h8 *>(a.dout + b * a.dosb + h * a.dosh + row * a.doss + 8 * part);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += (float)ov[e] * (float)dv[e];
    }
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (row < S && part == 0) {
        a.delta[(int64_t)bh * S + row] = sum;
        if (a.lse) {
            const float l2 = a.lse[b * a.lsb + h * a.lsh + row] * LOG2E;
            a.lse2[(int64_t)bh * S + row] = l2;
            store_row_terms(a, bh, row, l2, sum);
        }
    }
}

// ---------------------------------------------------------------------------
// dQ pass (+ delta)
// ---------------------------------------------------------------------------
constexpr int DQ_NW = 4;
constexpr int DQ_QB = 2;                    // 32-query blocks per wave
constexpr int DQ_KT = 64;                   // keys per tile
constexpr int DQ_QWG = DQ_NW * 32 * DQ_QB;  // 256 queries per workgroup
constexpr int QP_NST = 4;   // LDS stages: a pair of key tiles read, the next pair in flight

// 256 queries per workgroup, 64 per wave (two 32-query blocks), 64-key tiles
// taken 32 keys (kb) at a time, in order: S and dP of both query blocks from
// one pass over the K / V row fragments (each fragment read from LDS feeds two
// MFMAs), dS, then dQ of both blocks from one pass over the K^T fragments.
// The loop is not pipelined inside the wave -- the other workgroup's wave on
// the same SIMD overlaps its matrix and vector work.  Tiles go in pairs with
// one barrier per pair: while two tiles are read, the next two are in
// flight.  (A pipelined form that interleaved neighbouring 32 x 32 units
// inside the wave, each reading its fragments itself, was 2% slower at
// S = 4096 and 4% at S = 512.)
//
// DMASK (dropout with a.drop_mask): the keep bits come from the words the
// forward wrote (two per query and key tile, moved into LDS with the tile)
// instead of the hash.
//
// NARROW: one 32-query block per wave (128 queries per workgroup), the same
// in-order tile body, NSK = 2 or 3 LDS stages with one barrier per tile, and
// at most 128 or 168 registers per lane, so that four or three workgroups
// (waves per SIMD) share a CU and cover each other's latencies.
#ifndef FA2_DQ_NARROW_WAVES
#define FA2_DQ_NARROW_WAVES 3
#endif
constexpr int DQ_NARROW_WAVES = FA2_DQ_NARROW_WAVES;
static_assert(DQ_NARROW_WAVES == 3 || DQ_NARROW_WAVES == 4, "three or four narrow waves per SIMD");

template <bool CAUSAL, bool DROPOUT, bool DMASK, bool NARROW = false>
__global__ __launch_bounds__(256, NARROW ? DQ_NARROW_WAVES : 2) void bwd_dq_pipe_kernel(const BwdArgs a) {
    static_assert(!DMASK || DROPOUT, "keep-bit words only with dropout");
    constexpr int QB = NARROW ? 1 : DQ_QB;            // 32-query blocks per wave
    constexpr int QWG = DQ_NW * 32 * QB;              // queries per workgroup
    constexpr int NSK = NARROW ? (DQ_NARROW_WAVES == 4 ? 2 : 3) : QP_NST;   // LDS stages
    __shared__ __attribute__((aligned(16))) h8 sKV[NSK][2][DQ_KT * 8];
    // DMASK: per stage and wave, the words of its 64 queries (32 when NARROW)
    // for halves g2 = 0, 1.
    __shared__ __attribute__((aligned(16))) uint32_t sMQ[DMASK ? NSK : 1][DQ_NW][2][64];
    // Each lane's four transfer offsets of a full tile (K rows i = 0, 1, then
    // V rows), 1 KB per wave.
    typedef uint32_t u4x __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) u4x sOff[DQ_NW * 64];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, c = lane & 31, g2 = lane >> 5;
    const int S = a.S;
    const int BH = a.B * a.H;
    const int nqblk = (S + QWG - 1) / QWG;
    int qslot, bh;
    query_block_order(blockIdx.x, BH, nqblk, a.hgroup, qslot, bh);
    const int qblk = nqblk - 1 - qslot;   // heaviest (last) query blocks first
    const int b = bh / a.H, h = bh - b * a.H;

    const _Float16 *Qp = a.q + b * a.qsb + h * a.qsh;
    const _Float16 *Kp = a.k + b * a.ksb + h * a.ksh;
    const _Float16 *Vp = a.v + b * a.vsb + h * a.vsh;
    const _Float16 *Op = a.o + b * a.osb + h * a.osh;
    const _Float16 *dOp = a.dout + b * a.dosb + h * a.dosh;
    const float *Lp = a.lse + b * a.lsb + h * a.lsh;
    _Float16 *dQp = a.dq + b * a.dqsb + h * a.dqsh;
    float *Dp = a.delta + (int64_t)bh * S;

    const int q_wg0 = qblk * QWG;
    const int qw0 = q_wg0 + wave * 32 * QB;
    const float scale2 = a.scale2;

    // The first key tiles go out before the wave's Q, dO and O rows are
    // loaded: the delta computation waits for those rows, and with the
    // transfers already in flight the two round trips overlap.
    const int kend = CAUSAL ? min(S, q_wg0 + QWG) : S;
    const int ntiles = (kend + DQ_KT - 1) / DQ_KT;
    // Last key tile of this wave (-1: none).  The wave's first query is a
    // multiple of the tile size, so only that tile can need a mask.
    const int tlast = (qw0 >= S) ? -1 : CAUSAL ? (min(qw0 + 32 * QB, S) - 1) / DQ_KT : ntiles - 1;

    // Stage of tile t (t >= 0; unsigned, so a power-of-two count is a mask).
    auto stage_of = [](int t) FA2_INLINE { return (int)((uint32_t)t % (uint32_t)NSK); };
    // Tile loader (direct global->LDS transfers): wave w moves transfers
    // j = 2w, 2w+1 of the K and the V tile; lane L of transfer j lands at
    // chunk position 64j + L = 8*row + (L & 7), row = 8j + (L >> 3), and
    // fetches logical chunk (L & 7) ^ swz_both(row) of key row k0 + row (rows
    // past S: row S - 1, masked on use).
    // The offsets of a full tile are fixed: computed once, kept in an LDS
    // slot of the wave and read back with one ds_read_b128 per tile (the
    // kernel has no registers to hold them across the loop; recomputing them
    // every tile cost ~25 VALU instructions).  The last, partial tile
    // recomputes them from the lane index, re-read through an opaque move so
    // that nothing derived from it stays live across the tile loop.
    auto tile_offsets = [&](int k0, uint32_t(&ko)[2], uint32_t(&vo)[2]) FA2_INLINE {
        int ln;
        asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
        const int lrow = ln >> 3;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ch = (ln & 7) ^ swz_both(lrow + 8 * i);
            const int row = min(k0 + 8 * (2 * wave + i) + lrow, S - 1) - k0;
            ko[i] = (mul_u24((uint32_t)a.kss, (uint32_t)row) + 8 * ch) * 2u;   // strides < 2^24 (host check)
            vo[i] = (mul_u24((uint32_t)a.vss, (uint32_t)row) + 8 * ch) * 2u;
        }
    };
    // Tiles are issued in order, once each: issue_next() sends the next tile
    // (the callers' index tests only decide whether there is one).  Scalar
    // running addresses (global tile bases, LDS stage) advance by a constant
    // per tile.
    uint64_t gk = (uint64_t)(uintptr_t)Kp, gv = (uint64_t)(uintptr_t)Vp;
    const uint64_t k_step = (uint64_t)DQ_KT * a.kss * 2, v_step = (uint64_t)DQ_KT * a.vss * 2;
    int kn = 0;          // first key of the next tile to issue
    uint32_t stn = 0;    // its stage
    const uint32_t lds_kv = lds_addr(&sKV[0][0][0]) + 2048u * (uint32_t)wave;
    // DMASK: the wave's 64 (NARROW: 32) words per half g2 of each tile (rows
    // past S are within the mask's padded rows), 4 bytes per lane.
    const uint32_t lds_mq = lds_addr(&sMQ[0][wave][0][0]);
    {
        // (With S < DQ_KT every tile is partial and recomputes its offsets,
        // so the clamped values stored then go unread.)
        uint32_t ko[2], vo[2];
        tile_offsets(0, ko, vo);
        sOff[64 * wave + lane] = u4x{ko[0], ko[1], vo[0], vo[1]};
    }
    auto issue_next = [&]() FA2_INLINE {
        uint32_t ko[2], vo[2];
        if (kn + DQ_KT > S) {
            tile_offsets(kn, ko, vo);
        } else {
            // An opaque slot address: the read stays in the loop instead of
            // being hoisted into four live registers.
            uint32_t oa = lds_addr(&sOff[64 * wave]) + 16u * (uint32_t)lane;
            asm volatile("" : "+v"(oa));
            const u4x ov = *reinterpret_cast<const __attribute__((address_space(3))) u4x *>(oa);
            ko[0] = ov[0];
            ko[1] = ov[1];
            vo[0] = ov[2];
            vo[1] = ov[3];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t d = lds_kv + stn * (uint32_t)sizeof(sKV[0]) + 1024u * (uint32_t)i;
            lds_dma16_at(gk, ko[i], d);
            lds_dma16_at(gv, vo[i], d + (uint32_t)sizeof(sKV[0][0]));
        }
        if (DMASK) {
#pragma unroll
            for (int half = 0; half < 2; ++half)
                lds_dma4_at((uint64_t)(uintptr_t)(a.drop_mask + dmask_word(CAUSAL, bh, S, kn / DQ_KT, half, qw0)),
                            4u * (uint32_t)(NARROW ? (lane & 31) : lane),   // NARROW: 32 words, lanes 32.. repeat
                            lds_mq + stn * (uint32_t)sizeof(sMQ[0]) + 256u * (uint32_t)half);
        }
        gk += k_step;
        gv += v_step;
        kn += DQ_KT;
        stn = (stn + 1 == NSK) ? 0 : stn + 1;
    };
#pragma unroll
    for (int t = 0; t < NSK - 1; ++t)
        if (t < ntiles) issue_next();

    // Resident Q^T / dO^T operands, delta and log2-scaled LSE of the wave's
    // queries (rows past S: row S - 1 and LSE = +inf, so P = dS = 0).
    h8 qf[QB][4], dof[QB][4];
    float lse2[QB], dl[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int q = qw0 + 32 * qb + c;
        const bool valid = q < S;
        const int qr = min(q, S - 1);
        float part = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int d0 = 16 * st + 8 * g2;
            const h8 qv = *reinterpret_cast<const h8 *>(Qp + (int64_t)qr * a.qss + d0);
            const h8 dv = *reinterpret_cast<const h8 *>(dOp + (int64_t)qr * a.doss + d0);
            const h8 ov = *reinterpret_cast<const h8 *>(Op + (int64_t)qr * a.oss + d0);
            qf[qb][st] = neg_h8_if(qv, a.negate);
            dof[qb][st] = dv;
#pragma unroll
            for (int e = 0; e < 8; ++e) part += (float)ov[e] * (float)dv[e];
        }
        dl[qb] = part + xor32(part);
        lse2[qb] = valid ? Lp[qr] * LOG2E : INFINITY;
        if (valid && g2 == 0) {   // for the dK/dV pass
            Dp[q] = dl[qb];
            a.lse2[(int64_t)bh * S + q] = lse2[qb];
            store_row_terms(a, bh, q, lse2[qb], dl[qb]);
        }
    }

    f16x dq[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        dq[qb][0] = zero16();
        dq[qb][1] = zero16();
    }
    // Without dropout, dP^T - delta comes out of the MFMA chain: the dP
    // accumulator starts at -delta (the lane's query: the same value in all
    // 16 elements, 16 moves), so dS = P * acc needs no subtraction.  (An
    // extra bf16 MFMA step adding -delta from three bf16 parts costs 2% more
    // time in this pass, and 16 subtractions per block 2%.)

    // LDS read offsets: K / V rows 32*kb + c at logical chunk 2*st + g2, and
    // K^T through transposing reads (d block db, row half hi).
    int roff[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) roff[st] = c * 128 + (((2 * st + g2) ^ swz_both(c)) << 4);
    int toff[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) toff[db][hi] = tr_both_off(32 * db, hi);
    auto rrow = [&](int stage, int which, int kb, int st) FA2_INLINE {
        return *reinterpret_cast<const h8 *>(reinterpret_cast<const char *>(sKV[stage][which]) + roff[st] +
                                             kb * 32 * 128);
    };
    auto trk = [&](int stage, int kb, int db, int hh) FA2_INLINE {
        return tr_read8_both(reinterpret_cast<const _Float16 *>(sKV[stage][0]), toff[db][0], toff[db][1],
                             32 * kb + 16 * hh);
    };

    // Keys past S and, causal, after the query -> -inf.  key = t*KT + 32*kb +
    // 4*g2 + (8*(r>>2) + (r&3)), compared as a constant against a per-lane bound.
    auto need_mask = [&](int t) FA2_INLINE {
        return (t * DQ_KT + DQ_KT > S) || (CAUSAL && t * DQ_KT + DQ_KT - 1 > qw0);
    };
    auto mask = [&](int t, int kb, int qb, f16x &s) FA2_INLINE {
        const int q = qw0 + 32 * qb + c;
        const int bound = (CAUSAL ? min(q, S - 1) : S - 1) - t * DQ_KT - 32 * kb - 4 * g2;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) > bound) s[r] = -INFINITY;
    };
    // dS of element r of unit (t, kb, qb) from its score and dP value.
    // (Without dropout g is dP - delta already.)
    // DMASK: mw is the unit's keep word (query qw0 + 32*qb + c, tile t, half
    // g2), whose bit 31 - (16*kb + r) is element r's.
    auto ds_of = [&](float sv, float g, int t, int kb, int qb, int r, uint32_t mw) FA2_INLINE {
        const float p = __builtin_amdgcn_exp2f(fmaf(sv, scale2, -lse2[qb]));
        if (!DROPOUT) return p * g;
        const int key = t * DQ_KT + 32 * kb + 8 * (r >> 2) + 4 * g2 + (r & 3);
        // The keep decision selects the multiplier 1/(1-p) or 0 (from the
        // word: keep_multiplier; from the hash: a select), the same form on
        // both paths so that they give the same bits.
        const float m = DMASK ? keep_multiplier(mw, 31 - (16 * kb + r), a.inv_keep)
                              : (dropout_keep_hashed(dropout_row_part(a.seed, qw0 + 32 * qb + c, (uint32_t)bh) ^
                                                         dropout_col_term(key),
                                                     a.drop_thr)
                                     ? a.inv_keep
                                     : 0.f);
        return p * (g * m - dl[qb]);
    };
    auto keep_word = [&](int t, int qb) FA2_INLINE -> uint32_t {
        return DMASK ? sMQ[DMASK ? stage_of(t) : 0][wave][g2][32 * qb + c] : 0u;
    };
    auto ds_form = [&](int t, int kb, int qb, const f16x &s, const f16x &dp, h8(&dsb)[2]) FA2_INLINE {
        f16x x;
        const uint32_t mw = keep_word(t, qb);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = ds_of(s[r], dp[r], t, kb, qb, r, mw);
        dsb[0] = acc_to_h8(x, 0);
        dsb[1] = acc_to_h8(x, 1);
    };

    // Query block qb's units keep S, dP and dS in role qb (A: 0, B: 1).
    f16x sA, dpA, sB, dpB;
    h8 dsA[2], dsB[2];
    constexpr int TPT = DMASK ? 6 : 4;   // transfers per tile and wave
    if constexpr (NARROW) {
        // One query block: per 32 keys (kb) of tile t, S and dP, dS, then dQ.
        // NSK stages: tile t is read while tiles t+1 .. t+NSK-1 are in
        // flight; the end of tile t waits for tile t+1 (later tiles' transfers
        // may still be pending), joins the barrier after which no wave reads
        // stage t % NSK any more, and sends tile t+NSK there.
        auto wait_tiles = [&](int n) FA2_INLINE {   // at most n tiles' transfers pending
            if (n <= 0) vm_wait<0>();
            else if (n == 1) vm_wait<TPT>();
            else vm_wait<2 * TPT>();
        };
        if (NSK - 1 < ntiles) issue_next();   // the last stage's tile (the prologue sent the others)
        wait_tiles(min(NSK - 1, ntiles - 1));
        lds_barrier();                         // tile 0 landed for every wave
        // Unrolled over the NSK stages (every wave starts at tile 0 and tile t
        // sits in stage t % NSK), so that each copy's stage is a constant and
        // the operand reads address LDS through instruction offsets.
        for (int t0 = 0; t0 < ntiles; t0 += NSK) {
#pragma unroll
          for (int st = 0; st < NSK; ++st) {
            const int t = t0 + st;
            if (t >= ntiles) break;
            if (t <= tlast) {
                const bool m = need_mask(t);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    if (!DROPOUT) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) dpA[r] = -dl[0];
                    }
#pragma unroll
                    for (int sti = 0; sti < 4; ++sti) {
                        const h8 ka = rrow(st, 0, kb, sti), va = rrow(st, 1, kb, sti);
                        sA = sti == 0 ? mfma32_first(ka, qf[0][0]) : mfma32(ka, qf[0][sti], sA);
                        dpA = (sti == 0 && DROPOUT) ? mfma32_first(va, dof[0][0]) : mfma32(va, dof[0][sti], dpA);
                    }
                    if (m) {
                        FA2_COLD_BRANCH();
                        mask(t, kb, 0, sA);
                    }
                    ds_form(t, kb, 0, sA, dpA, dsA);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int db = 0; db < 2; ++db) dq[0][db] = mfma32(trk(st, kb, db, hh), dsA[hh], dq[0][db]);
                }
            }
            if (t + 1 < ntiles) {
                wait_tiles(min(NSK - 2, ntiles - 2 - t));   // tile t+1 landed
                lds_barrier();
                if (t + NSK < ntiles) issue_next();
            }
          }
        }
        vm_wait<0>();
        lds_barrier();   // every wave is done with the stages: the dQ staging reuses them
    } else {
        // Two query blocks: S and dP of both from one pass over the K / V row
        // fragments (each fragment read from LDS feeds two MFMAs), dS, then dQ
        // of both from one pass over the K^T fragments.
        // Tiles are computed in pairs with one barrier after each pair: while
        // tiles t-1, t are read, t+1, t+2 are in flight; the pair's end waits
        // for those two (every issued transfer) and refills the two stages
        // just read with tiles t+3, t+4.  Tile 3 goes out now.
        if (NSK - 1 < ntiles) issue_next();
        auto wait_pending = [&](int n) FA2_INLINE {
            if (n <= 0) vm_wait<0>();
            else if (n == 1) vm_wait<TPT>();
            else if (n == 2) vm_wait<2 * TPT>();
            else vm_wait<3 * TPT>();
        };
        wait_pending(min(NSK - 2, ntiles - 2));   // tiles 0 and 1 landed
        lds_barrier();
        // Unrolled over the four stages, as in the narrow loop.
        for (int t0 = 0; t0 < ntiles; t0 += NSK) {
#pragma unroll
          for (int st = 0; st < NSK; ++st) {
            const int t = t0 + st;
            if (t >= ntiles) break;
            if (t <= tlast) {
                const bool m = need_mask(t);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    if (!DROPOUT) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            dpA[r] = -dl[0];
                            dpB[r] = -dl[QB - 1];
                        }
                    }
#pragma unroll
                    for (int sti = 0; sti < 4; ++sti) {
                        const h8 ka = rrow(st, 0, kb, sti), va = rrow(st, 1, kb, sti);
                        sA = sti == 0 ? mfma32_first(ka, qf[0][0]) : mfma32(ka, qf[0][sti], sA);
                        sB = sti == 0 ? mfma32_first(ka, qf[QB - 1][0]) : mfma32(ka, qf[QB - 1][sti], sB);
                        dpA = (sti == 0 && DROPOUT) ? mfma32_first(va, dof[0][0]) : mfma32(va, dof[0][sti], dpA);
                        dpB = (sti == 0 && DROPOUT) ? mfma32_first(va, dof[QB - 1][0])
                                                    : mfma32(va, dof[QB - 1][sti], dpB);
                    }
                    if (m) {
                        FA2_COLD_BRANCH();
                        mask(t, kb, 0, sA);
                        mask(t, kb, QB - 1, sB);
                    }
                    ds_form(t, kb, 0, sA, dpA, dsA);
                    ds_form(t, kb, QB - 1, sB, dpB, dsB);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int db = 0; db < 2; ++db) {
                            const h8 kt = trk(st, kb, db, hh);
                            dq[0][db] = mfma32(kt, dsA[hh], dq[0][db]);
                            dq[QB - 1][db] = mfma32(kt, dsB[hh], dq[QB - 1][db]);
                        }
                }
            }
            if ((t & 1) && t < ntiles - 1) {   // the end of a pair, not the last tile
                vm_wait<0>();                  // tiles t+1, t+2 (the next pair) landed
                lds_barrier();
                if (t + 3 < ntiles) issue_next();
                if (t + 4 < ntiles) issue_next();
            }
          }
        }
    }

    // dQ rows leave through LDS (store_rows_f16), 4 KB per 32-query block.
    // NARROW: after the final barrier every stage is idle; wave w uses
    // bytes 4096*w on.  Otherwise the last pair (or single last tile) has no
    // barrier after it, so other waves may still read the stages of tiles
    // ntiles-2 and ntiles-1; stages ntiles % 4 and (ntiles + 1) % 4 are idle
    // (their last reads precede an earlier barrier, no later transfer
    // refilled them, and every transfer has landed): waves 0, 1 use the
    // first, waves 2, 3 the second.
    static_assert(NARROW ? sizeof(sKV) >= DQ_NW * 4096 : (NSK == 4 && QB == 2 && sizeof(sKV[0]) == 16384),
                  "dQ staging layout");
    const float sc = a.scale;
    const bool dq16 = ((a.dqsb | a.dqsh | a.dqss) & 7) == 0;
    char *const stg = NARROW ? reinterpret_cast<char *>(&sKV[0][0][0]) + 4096 * wave
                             : reinterpret_cast<char *>(sKV[stage_of(ntiles + (wave >> 1))]) + 8192 * (wave & 1);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
        store_rows_f16(dq[qb][0], dq[qb][1], sc, stg + 4096 * qb, dQp + (int64_t)(qw0 + 32 * qb) * a.dqss, a.dqss,
                       S - (qw0 + 32 * qb), dq16);
}

// ---------------------------------------------------------------------------
// dK / dV pass, software pipelined (the default backward's second kernel)
// ---------------------------------------------------------------------------
constexpr int KP_NW = 4;
constexpr int KP_QT = 32;             // queries per tile
constexpr int KP_KWG = KP_NW * 32;    // keys per workgroup
#ifndef FA2_KV_NST
#define FA2_KV_NST 4
#endif
constexpr int KP_NST = FA2_KV_NST;    // LDS stages: tiles t-1, t, t+1 resident, t+2 .. in flight (4..6)
static_assert(KP_NST >= 4 && KP_NST <= 6, "dK/dV stages");
// FOLD: the chunk (0..3) of a steady step in which the next tile's row terms
// are read from LDS into its S and dP accumulators (two chunks ahead of their
// first MFMA, so the reads are done by then).
#ifndef FA2_KV_CINIT_CHUNK
#define FA2_KV_CINIT_CHUNK 2
#endif

// A workgroup owns 128 keys (32 per wave; K^T and V^T stay in registers) and
// streams 32-query tiles: Q and dO by direct global->LDS transfers into
// tiles swizzled so that both their row reads (S = Q K^T, dP = dO V^T) and
// their transposed reads (dV += dO^T P, dK += Q^T dS) are free of bank
// conflicts, and the tile's log2-scaled LSE and delta by one 4-byte transfer.
// Step t issues the dK/dV MFMAs of tile t-1 and the S/dP MFMAs of tile t+1
// while the VALU forms P and dS of tile t (reference @ None:
// csrc/flash_attn_v100/flash_attn_v100_bwd.cu:300-470 computes the same
// quantities per key tile).
//
// FOLD (no dropout; the host also requires scale2 >= 1e-20): the row terms
// -lse2/scale2 and -delta (fp32, written by the dQ or delta pass) are the
// initial values of the S and dP accumulators -- the first MFMA of each chain
// takes them as its C operand -- so P = exp2(S*scale2) and dS = P * dP take no
// per-element row statistics and no subtraction.  Otherwise the tile's lse2
// and delta are read from LDS per element.
//
// DMASK (dropout with a.drop_mask): the keep bits come from the words the
// forward wrote: per 32-query tile, the words of both 64-key tiles of the
// workgroup's keys (4 runs of 32 words), moved into LDS by wave 1; each lane
// tests one bit position of the words of its 16 query rows.
template <bool CAUSAL, bool DROPOUT, bool FOLD, bool DMASK>
__device__ __forceinline__ void dkv_block(const BwdArgs &a, const int kblk, const int bh) {
    static_assert(!(FOLD && DROPOUT), "the folded row terms assume no dropout");
    static_assert(!DMASK || DROPOUT, "keep-bit words only with dropout");
    __shared__ __attribute__((aligned(16))) h8 sQD[KP_NST][2][KP_QT * 8];   // Q, dO tiles (4 KB each)
    // Per stage: lse2[32], delta[32] (fp32); FOLD: the row terms -lse2/scale2
    // and -delta in the same places.
    __shared__ __attribute__((aligned(16))) float sLD[KP_NST][2 * KP_QT];
    // DMASK: per stage, run s = 2*i + g2' holds the 32 words of 64-key tile
    // 2*kblk + i, half g2' (and a copy from the transfer's upper 32 lanes).
    __shared__ __attribute__((aligned(16))) uint32_t sDM[DMASK ? KP_NST : 1][256];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, c = lane & 31, g2 = lane >> 5;
    const int S = a.S;
    const int BH = a.B * a.H;
    const int b = bh / a.H, h = bh - b * a.H;

    const _Float16 *Qp = a.q + b * a.qsb + h * a.qsh;
    const _Float16 *Kp = a.k + b * a.ksb + h * a.ksh;
    const _Float16 *Vp = a.v + b * a.vsb + h * a.vsh;
    const _Float16 *dOp = a.dout + b * a.dosb + h * a.dosh;
    _Float16 *dKp = a.dk + b * a.dksb + h * a.dksh;
    _Float16 *dVp = a.dv + b * a.dvsb + h * a.dvsh;

    const int k_wg0 = kblk * KP_KWG;
    const int kw0 = k_wg0 + 32 * wave;    // this wave's keys kw0 .. kw0 + 31
    const int key = kw0 + c;               // this lane's key
    const float scale2 = a.scale2;

    // K^T / V^T B operands of d-step st: lane holds K[key][16*st + 8*g2 + e].
    // Keys past S read row S - 1; their dK/dV columns are never stored.
    h8 kf[4], vf[4];
    {
        const int kr = min(key, S - 1);
        const _Float16 *krow = Kp + (int64_t)kr * a.kss + 8 * g2;
        const _Float16 *vrow = Vp + (int64_t)kr * a.vss + 8 * g2;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const h8 kv = *reinterpret_cast<const h8 *>(krow + 16 * st);
            kf[st] = neg_h8_if(kv, a.negate);
            vf[st] = *reinterpret_cast<const h8 *>(vrow + 16 * st);
        }
    }

    const int q_start = CAUSAL ? k_wg0 : 0;
    const int ntiles = (k_wg0 < S) ? (S - q_start + KP_QT - 1) / KP_QT : 0;
    // First tile this wave computes (ntiles: none).  Causal: the tile holding
    // the wave's diagonal; earlier tiles lie entirely above it.
    const int tfirst = (kw0 >= S) ? ntiles : CAUSAL ? (kw0 - q_start) / KP_QT : 0;

    // Tile loader.  Q and dO tiles are 256 chunks = 4 transfers each; wave w
    // moves transfer w of both: lane L lands at chunk position 64w + L =
    // 8*row + (L & 7), row = 8w + (L >> 3), and fetches logical chunk
    // (L & 7) ^ swz_both(row) of query row q0 + row (rows past S: row S - 1,
    // masked on use).  Wave 0 also moves the tile's lse2 (lanes 0..31) and
    // delta (lanes 32..63) from the workspace, where lse2 = delta + B*H*S.
    // FOLD: wave 0 moves the tile's 256-byte block of row terms instead.
    const int trow = 8 * wave + (lane >> 3);
    const int tch = (lane & 7) ^ swz_both(trow);
    auto tile_offsets = [&](int q0, uint32_t &qo, uint32_t &doo) FA2_INLINE {
        const int row = min(q0 + trow, S - 1) - q0;
        qo = (mul_u24((uint32_t)a.qss, (uint32_t)row) + 8 * tch) * 2u;     // strides < 2^24 (host check)
        doo = (mul_u24((uint32_t)a.doss, (uint32_t)row) + 8 * tch) * 2u;
    };
    // Stage of tile t (t >= 0; unsigned, so a power-of-two count is a mask).
    auto stage_of = [](int t) FA2_INLINE { return (int)((uint32_t)t % (uint32_t)KP_NST); };
    uint32_t qoff0, dooff0;
    tile_offsets(0, qoff0, dooff0);
    const uint32_t ldoff = ((lane < 32) ? (uint32_t)BH * (uint32_t)S * 4u : 0u) + 4u * (uint32_t)(lane & 31);
    // Tiles are issued in order, once each: issue_next() sends the next tile
    // (the callers' index tests only decide whether there is one).  Scalar
    // running addresses (global tile bases, LDS stage) advance by a constant
    // per tile instead of being recomputed with 64-bit multiplies at every
    // transfer.
    uint64_t gq = (uint64_t)(uintptr_t)(Qp + (int64_t)q_start * a.qss);
    uint64_t gdo = (uint64_t)(uintptr_t)(dOp + (int64_t)q_start * a.doss);
    uint64_t gld = FOLD ? (uint64_t)(uintptr_t)(a.rowterm + row_term_word(S, bh, q_start, 0))
                        : (uint64_t)(uintptr_t)(a.delta + (int64_t)bh * S + q_start);
    const uint32_t ldoff_t = FOLD ? 4u * (uint32_t)lane : ldoff;
    const uint64_t dq_step = (uint64_t)KP_QT * a.qss * 2, ddo_step = (uint64_t)KP_QT * a.doss * 2;
    int qn = q_start;          // first query of the next tile to issue
    uint32_t stn = 0;          // its stage
    const uint32_t lds_qd = lds_addr(&sQD[0][0][0]) + 1024u * (uint32_t)wave, lds_ld = lds_addr(&sLD[0][0]);
    // DMASK: lane L of wave 1's transfer moves words 4*(L & 7) .. +3 of run
    // s = (L & 31) >> 3, i.e. of 64-key tile 2*kblk + (s >> 1), half s & 1,
    // at word s * dmask_run(...) past the tile's first run (both tiles of the
    // block have runs of one length; lanes 32..63 repeat lanes 0..31).
    const uint32_t dmoff = 4u * (uint32_t)(((lane & 31) >> 3) * dmask_run(CAUSAL, S, 2 * kblk) + 4 * (lane & 7));
    const uint32_t lds_dm = lds_addr(&sDM[0][0]);
    auto issue_next = [&]() FA2_INLINE {
        uint32_t qo = qoff0, doo = dooff0;
        if (qn + KP_QT > S) tile_offsets(qn, qo, doo);
        lds_dma16_at(gq, qo, lds_qd + stn * (uint32_t)sizeof(sQD[0]));
        lds_dma16_at(gdo, doo, lds_qd + stn * (uint32_t)sizeof(sQD[0]) + (uint32_t)sizeof(sQD[0][0]));
        if (wave == 0) lds_dma4_at(gld, ldoff_t, lds_ld + stn * (uint32_t)sizeof(sLD[0]));
        if (DMASK && wave == 1)
            lds_dma16_at((uint64_t)(uintptr_t)(a.drop_mask + dmask_word(CAUSAL, bh, S, 2 * kblk, 0, qn)), dmoff,
                         lds_dm + stn * (uint32_t)sizeof(sDM[0]));
        gq += dq_step;
        gdo += ddo_step;
        gld += FOLD ? 2 * KP_QT * sizeof(float) : KP_QT * sizeof(float);
        qn += KP_QT;
        stn = (stn + 1 == KP_NST) ? 0 : stn + 1;
    };
#pragma unroll
    for (int t = 0; t < KP_NST - 1; ++t)
        if (t < ntiles) issue_next();
    // Transfers per tile and wave: 2, plus 1 for wave 0 (and, DMASK, for
    // wave 1).  Wait until at most n tiles' transfers are pending.
    const bool three = wave == 0 || (DMASK && wave == 1);
    auto wait_tiles = [&](int n) FA2_INLINE {
        if (n <= 0) vm_wait<0>();
        else if (n == 1) { if (three) vm_wait<3>(); else vm_wait<2>(); }
        else if (n == 2) { if (three) vm_wait<6>(); else vm_wait<4>(); }
        else { if (three) vm_wait<9>(); else vm_wait<6>(); }
    };
    auto tile_end = [&](int t) FA2_INLINE {
        // tile t+2 landed (tiles up to t+NST-2 issued); stage of tile t-1 free
        wait_tiles(min(KP_NST - 4, ntiles - 1 - (t + 2)));
        lds_barrier();
        if (t + KP_NST - 1 < ntiles) issue_next();
    };

    f16x dk[2] = {zero16(), zero16()}, dv[2] = {zero16(), zero16()};   // dK^T, dV^T (d blocks)

    // LDS read offsets.  Row reads (A operands of S and dP): query row c,
    // logical chunk 2*st + g2.  Transposed reads: d block db, row half hi.
    int roff[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) roff[st] = c * 128 + (((2 * st + g2) ^ swz_both(c)) << 4);
    int toff[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) toff[db][hi] = tr_both_off(32 * db, hi);
    auto rread = [&](int stage, int which, int st) FA2_INLINE {
        return *reinterpret_cast<const h8 *>(reinterpret_cast<const char *>(sQD[stage][which]) + roff[st]);
    };
    auto tread = [&](int stage, int which, int db, int hh) FA2_INLINE {
        return tr_read8_both(reinterpret_cast<const _Float16 *>(sQD[stage][which]), toff[db][0], toff[db][1],
                             16 * hh);
    };
    // FOLD: the initial accumulator of the S (which = 0) or dP (which = 1)
    // chain of the tile in `stage`: element 4i + j holds the row term of query
    // row 8i + 4*g2 + j (four 16-byte reads, the same for every lane of a half).
    auto cinit = [&](int stage, int which) FA2_INLINE {
        f16x v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f4 x = *reinterpret_cast<const f4 *>(&sLD[stage][KP_QT * which + 8 * i + 4 * g2]);
#pragma unroll
            for (int j = 0; j < 4; ++j) v[4 * i + j] = x[j];
        }
        return v;
    };

    // S = Q K^T and dP = dO V^T of the tile in `stage`: rows = the tile's
    // queries 8i + 4*g2 + j, column = this lane's key.
    auto sdp = [&](int stage, f16x &s, f16x &dp) FA2_INLINE {
        h8 nq = rread(stage, 0, 0), nd = rread(stage, 1, 0);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const h8 fq = nq, fd = nd;
            if (st < 3) {
                nq = rread(stage, 0, st + 1);
                nd = rread(stage, 1, st + 1);
            }
            if (st == 0 && FOLD) {
                s = mfma32(fq, kf[0], cinit(stage, 0));
                dp = mfma32(fd, vf[0], cinit(stage, 1));
            } else if (st == 0) {
                s = mfma32_first(fq, kf[0]);
                dp = mfma32_first(fd, vf[0]);
            } else {
                s = mfma32(fq, kf[st], s);
                dp = mfma32(fd, vf[st], dp);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // dV^T += dO^T P and dK^T += Q^T dS over the tile in `stage`.
    auto dkdv = [&](int stage, const h8(&pb)[2], const h8(&dsb)[2]) FA2_INLINE {
#pragma unroll
        for (int i = 0; i < 4; ++i) {   // (db, hh) = (i >> 1, i & 1)
            const int db = i >> 1, hh = i & 1;
            dv[db] = mfma32(tread(stage, 1, db, hh), pb[hh], dv[db]);
            dk[db] = mfma32(tread(stage, 0, db, hh), dsb[hh], dk[db]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // P and dS of element r (query row q) of a tile, from its score s, dP
    // value g, lse2 l and delta dl.  Dropout: dV takes the kept, rescaled P;
    // dS = P * (dP * keep / (1-p) - delta).
    // FOLD: s and g already hold S - lse2/scale2 and dP - delta.
    // DMASK: mw is the keep word of the element's query row, whose bit kbit
    // is this lane's key (run dm_run of the tile's words).
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const int kbit = 31 - (16 * (wave & 1) + 8 * ((c >> 4) & 1) + 4 * ((c >> 3) & 1) + (c & 3));
    const int dm_run = 2 * (wave >> 1) + ((c >> 2) & 1);
    // Hash path: the seed, head and key terms of this lane's key, once.
    const uint32_t hcol = DROPOUT && !DMASK ? dropout_col_part(a.seed, key, (uint32_t)bh) : 0u;
    auto pds = [&](float sv, float g, float l, float dl, int q, uint32_t mw, float &pd, float &ds) FA2_INLINE {
        if (FOLD) {
            pd = __builtin_amdgcn_exp2f(sv * scale2);
            ds = pd * g;
            return;
        }
        const float p = __builtin_amdgcn_exp2f(fmaf(sv, scale2, -l));
        if (DROPOUT) {
            if (DMASK) {
                pd = p * keep_multiplier(mw, kbit, a.inv_keep);   // p >= 0: p * 0 = +0, as the select
            } else {
                const bool keep = dropout_keep_hashed(hcol ^ dropout_row_term(q), a.drop_thr);
                pd = keep ? p * a.inv_keep : 0.f;
            }
            ds = pd * g - p * dl;
        } else {
            pd = p;
            ds = p * (g - dl);
        }
    };
    // The tile's lse2 / delta for this lane's rows 8i + 4*g2 + j.
    // (and, DMASK, their keep words)
    auto stats = [&](int stage, f4(&l4)[4], f4(&d4)[4], u4v(&m4)[4]) FA2_INLINE {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m4[i] = u4v{0u, 0u, 0u, 0u};
            if (FOLD) {   // unused
                l4[i] = f4{0.f, 0.f, 0.f, 0.f};
                d4[i] = l4[i];
                continue;
            }
            l4[i] = *reinterpret_cast<const f4 *>(&sLD[stage][8 * i + 4 * g2]);
            d4[i] = *reinterpret_cast<const f4 *>(&sLD[stage][KP_QT + 8 * i + 4 * g2]);
            if (DMASK) m4[i] = *reinterpret_cast<const u4v *>(&sDM[DMASK ? stage : 0][32 * dm_run + 8 * i + 4 * g2]);
        }
    };
    // General P / dS (first and last tiles): rows past S and, causal, keys
    // after the query are forced to exactly zero (their lse2 / delta may be
    // anything).
    auto pds_general = [&](int t, const f16x &s, const f16x &dp, h8(&pb)[2], h8(&dsb)[2]) FA2_INLINE {
        const int q0 = q_start + t * KP_QT;
        f4 l4[4], d4[4];
        u4v m4[4];
        stats(stage_of(t), l4, d4, m4);
        const int lo = key - q0 - 4 * g2;        // visible iff off >= lo (causal)
        const int hi = S - q0 - 4 * g2;          // and off < hi
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            f8 xp, xd;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int r = 8 * hh + e;
                const int off = 8 * (r >> 2) + (r & 3);
                float pd, ds;
                pds(s[r], dp[r], l4[r >> 2][r & 3], d4[r >> 2][r & 3], q0 + 4 * g2 + off, m4[r >> 2][r & 3], pd, ds);
                const bool vis = (!CAUSAL || off >= lo) && off < hi;
                xp[e] = vis ? pd : 0.f;
                xd[e] = vis ? ds : 0.f;
            }
            pb[hh] = __builtin_convertvector(xp, h8);
            dsb[hh] = __builtin_convertvector(xd, h8);
        }
    };
    // Steady step t (no masking: the tile is below the diagonal of every key
    // of this wave and not the last one): dK/dV of tile t-1 from (pb_p,
    // ds_p), S/dP of tile t+1 into (s_n, dp_n), P/dS of tile t from (s_c,
    // dp_c) into (pb_c, ds_c).  Eight chunks of two MFMAs and two elements.
    auto step_at = [&](int t, int sp, int sc_, int sn, f16x &s_n, f16x &dp_n, const h8(&pb_p)[2],
                       const h8(&ds_p)[2], const f16x &s_c, const f16x &dp_c, h8(&pb_c)[2],
                       h8(&ds_c)[2]) FA2_INLINE {
        const int q0 = q_start + t * KP_QT;
        f4 l4[4], d4[4];
        u4v m4[4];
        stats(sc_, l4, d4, m4);
        // chunk i < 4: dK/dV for (db, hh) = (i >> 1, i & 1); i >= 4: S/dP for d-step i - 4
        h8 n0 = tread(sp, 1, 0, 0), n1 = tread(sp, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const h8 f0 = n0, f1 = n1;
            if (i < 3) {
                n0 = tread(sp, 1, (i + 1) >> 1, (i + 1) & 1);
                n1 = tread(sp, 0, (i + 1) >> 1, (i + 1) & 1);
            } else if (i < 7) {
                n0 = rread(sn, 0, i - 3);
                n1 = rread(sn, 1, i - 3);
            }
            if (i < 4) {
                const int db = i >> 1, hh = i & 1;
                dv[db] = mfma32(f0, pb_p[hh], dv[db]);
                dk[db] = mfma32(f1, ds_p[hh], dk[db]);
                if (FOLD && i == FA2_KV_CINIT_CHUNK) {
                    s_n = cinit(sn, 0);
                    dp_n = cinit(sn, 1);
                }
            } else if (i == 4 && FOLD) {
                s_n = mfma32(f0, kf[0], s_n);
                dp_n = mfma32(f1, vf[0], dp_n);
            } else if (i == 4) {
                s_n = mfma32_first(f0, kf[0]);
                dp_n = mfma32_first(f1, vf[0]);
            } else {
                s_n = mfma32(f0, kf[i - 4], s_n);
                dp_n = mfma32(f1, vf[i - 4], dp_n);
            }
            // elements r = 2i, 2i + 1 of tile t
            f2 xp, xd;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int r = 2 * i + e;
                float pd, ds;
                pds(s_c[r], dp_c[r], l4[r >> 2][r & 3], d4[r >> 2][r & 3], q0 + 4 * g2 + 8 * (r >> 2) + (r & 3),
                    m4[r >> 2][r & 3], pd, ds);
                xp[e] = pd;
                xd[e] = ds;
            }
            const h2 hp = __builtin_convertvector(xp, h2), hd = __builtin_convertvector(xd, h2);
            // Consumed here: keeps the chunk's VALU work beside its MFMAs
            // (otherwise it is sunk past the tile's barrier to its use).
            asm volatile("" ::"v"(hp), "v"(hd));
            pb_c[i >> 2][(2 * i) & 7] = hp[0];
            pb_c[i >> 2][(2 * i + 1) & 7] = hp[1];
            ds_c[i >> 2][(2 * i) & 7] = hd[0];
            ds_c[i >> 2][(2 * i + 1) & 7] = hd[1];
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto step = [&](int t, f16x &s_n, f16x &dp_n, const h8(&pb_p)[2], const h8(&ds_p)[2], const f16x &s_c,
                    const f16x &dp_c, h8(&pb_c)[2], h8(&ds_c)[2]) FA2_INLINE {
        step_at(t, stage_of(t + KP_NST - 1), stage_of(t), stage_of(t + 1), s_n, dp_n, pb_p, ds_p, s_c, dp_c,
                pb_c, ds_c);
    };

    // Tile t keeps its S, dP, P, dS in role X = (t - tfirst) & 1.
    f16x sA, dpA, sB, dpB;
    h8 pbA[2], dsA[2], pbB[2], dsB[2];
    const int tl = ntiles - 1;
    // Initial wait: tiles 0 and 1 landed, tiles 2 .. NST-2 may be in flight.
    wait_tiles(min(KP_NST - 3, ntiles - 2));
    lds_barrier();
    for (int t = 0; t < min(tfirst, ntiles); ++t) tile_end(t);
    if (tfirst < ntiles) {
        // First tile: serial order, masked.
        const int t0 = tfirst;
        sdp(stage_of(t0), sA, dpA);
        pds_general(t0, sA, dpA, pbA, dsA);
        if (t0 + 1 < ntiles) sdp(stage_of(t0 + 1), sB, dpB);
        if (t0 == tl) dkdv(stage_of(t0), pbA, dsA);
        tile_end(t0);
        int t = t0 + 1;
        for (; t + 1 < tl; t += 2) {   // roles B (t) and A (t + 1)
            step(t, sA, dpA, pbA, dsA, sB, dpB, pbB, dsB);
            tile_end(t);
            step(t + 1, sB, dpB, pbB, dsB, sA, dpA, pbA, dsA);
            tile_end(t + 1);
        }
        if (t < tl) {                  // role B
            step(t, sA, dpA, pbA, dsA, sB, dpB, pbB, dsB);
            tile_end(t);
            ++t;
        }
        if (t == tl && tl > t0) {
            // Last tile: its S/dP sit in role (tl - t0) & 1; move them to A once.
            if ((tl - t0) & 1) {
                const f16x ts = sA, td = dpA;
                sA = sB; dpA = dpB; sB = ts; dpB = td;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const h8 tp = pbA[hh], tq = dsA[hh];
                    pbA[hh] = pbB[hh]; dsA[hh] = dsB[hh]; pbB[hh] = tp; dsB[hh] = tq;
                }
            }
            dkdv(stage_of(tl + KP_NST - 1), pbB, dsB);   // tile tl - 1
            pds_general(tl, sA, dpA, pbA, dsA);
            dkdv(stage_of(tl), pbA, dsA);
            tile_end(tl);
        }
    }

    // dK, dV rows leave through LDS (store_rows_f16): after the last tile's
    // barrier no wave reads the stages and no transfer is in flight, so wave
    // w uses 8 KB of them.
    static_assert(sizeof(sQD) >= KP_NW * 8192, "dK/dV staging fits in the stages");
    const float sc = a.scale;
    char *const stg = reinterpret_cast<char *>(&sQD[0][0][0]) + 8192 * wave;
    store_rows_f16(dk[0], dk[1], sc, stg, dKp + (int64_t)kw0 * a.dkss, a.dkss, S - kw0,
                   ((a.dksb | a.dksh | a.dkss) & 7) == 0);
    store_rows_f16(dv[0], dv[1], 1.f, stg + 4096, dVp + (int64_t)kw0 * a.dvss, a.dvss, S - kw0,
                   ((a.dvsb | a.dvsh | a.dvss) & 7) == 0);
}

// The dK/dV pass: workgroup L owns key blocks kp and nkb - 1 - kp of one
// (b, h) (the middle block alone when nkb is odd), run one after the other:
// under the causal mask their query ranges add up to the same length for
// every pair, so all workgroups carry equal work.  Without the mask, and
// with dropout, a workgroup owns one block.  With B*H a multiple of 8,
// workgroups are numbered so that the 8 XCDs (blockIdx % 8) each take whole
// heads, head after head: the workgroups one XCD runs at a time share a few
// heads' Q / dO rows in its L2.
template <bool CAUSAL, bool DROPOUT, bool FOLD, bool DMASK>
__global__ __launch_bounds__(256, 2) void bwd_dkv_pipe_kernel(const BwdArgs a) {
    const int BH = a.B * a.H;
    const int nkb = (a.S + KP_KWG - 1) / KP_KWG;
    // (With dropout the second copy of the block's code would spill.)
    const bool pair = CAUSAL && !DROPOUT && a.dkv_pair;
    const int nwg_head = pair ? (nkb + 1) / 2 : nkb;   // workgroups per head
    const int L = blockIdx.x;
    int j, bh;
    if (pair && (BH & 7) == 0) {
        const int xcd = L & 7, i = L >> 3;
        bh = 8 * (i / nwg_head) + xcd;
        j = i - (i / nwg_head) * nwg_head;
    } else {
        j = L / BH;
        bh = L - j * BH;
    }
    // Single blocks: j = 0, the heaviest under the causal mask, first.  Pairs
    // of short blocks (nkb <= 8: S <= 1024): every other workgroup runs its
    // short block first, so that the workgroups sharing a CU, which start
    // together and carry equal work, do not also reach their block change
    // (the next block's first loads, the previous one's stores) at the same
    // time.  Longer sequences keep one order: a head's workgroups then stream
    // the same query tiles at about the same time, which keeps them in L2.
    const bool swap = pair && nkb <= 8 && ((L >> 3) & 1);
    const int ja = swap ? nkb - 1 - j : j, jb = swap ? j : nkb - 1 - j;
    dkv_block<CAUSAL, DROPOUT, FOLD, DMASK>(a, ja, bh);
    if (pair && jb != ja) {
        // The first block's dK/dV staging reads must finish before the second
        // block's transfers land in the same LDS.  (Two inlined copies of the
        // block: a loop over both keeps values live across them and spills.)
        lds_barrier();
        dkv_block<CAUSAL, DROPOUT, FOLD, DMASK>(a, jb, bh);
    }
}

}  // namespace

hipError_t launch_bwd_delta(const BwdArgs &a, hipStream_t st) {
    const int nrb = (a.S + 31) / 32;
    hipLaunchKernelGGL(bwd_delta_kernel, dim3((unsigned)(nrb * a.B * a.H)), dim3(256), 0, st, a);
    return hipGetLastError();
}

// Sequences up to this length take the narrow dQ kernel (one query block per
// wave, three waves per SIMD); longer ones the two-block kernel, whose shared
// K / V fragments halve the LDS reads per MFMA.  Measured at B*S = 32k, H = 12:
// S = 512 7% faster narrow, S = 1024 2.5% faster, S = 4096 6.5% slower.
#ifndef FA2_DQ_NARROW_MAX_S
#define FA2_DQ_NARROW_MAX_S 1024
#endif

// Keep-bit words always take the two-block kernel: reading them, the narrow
// one needs more registers than three waves per SIMD leave.
// Workgroup order of the dQ pass (query_block_order): groups of 16 heads per
// XCD up to this length (measured at B*S = 32k, H = 12: S = 512 3.5% faster;
// S = 1024 4.5% and S = 2048 11% slower), the plain order beyond.
#ifndef FA2_DQ_GROUP_MAX_S
#define FA2_DQ_GROUP_MAX_S 512
#endif

template <bool NARROW>
static void launch_dq_t(const BwdArgs &a_in, bool causal, bool dropout, hipStream_t st) {
    BwdArgs a = a_in;
    a.hgroup = (a.B * a.H) % 8 == 0 && a.S <= FA2_DQ_GROUP_MAX_S ? 16 : 0;
    const int qwg = NARROW && !(dropout && a.drop_mask != nullptr) ? DQ_NW * 32 : DQ_QWG;
    const dim3 grid((unsigned)((a.S + qwg - 1) / qwg * a.B * a.H)), block(256);
    const bool dmask = dropout && a.drop_mask != nullptr;
    if (causal) {
        if (dmask)
            hipLaunchKernelGGL((bwd_dq_pipe_kernel<true, true, true, false>), grid, block, 0, st, a);
        else if (dropout)
            hipLaunchKernelGGL((bwd_dq_pipe_kernel<true, true, false, NARROW>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((bwd_dq_pipe_kernel<true, false, false, NARROW>), grid, block, 0, st, a);
    } else {
        if (dmask)
            hipLaunchKernelGGL((bwd_dq_pipe_kernel<false, true, true, false>), grid, block, 0, st, a);
        else if (dropout)
            hipLaunchKernelGGL((bwd_dq_pipe_kernel<false, true, false, NARROW>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((bwd_dq_pipe_kernel<false, false, false, NARROW>), grid, block, 0, st, a);
    }
}

hipError_t launch_bwd_dq(const BwdArgs &a, bool causal, bool dropout, hipStream_t st) {
    if (a.S <= FA2_DQ_NARROW_MAX_S)
        launch_dq_t<true>(a, causal, dropout, st);
    else
        launch_dq_t<false>(a, causal, dropout, st);
    return hipGetLastError();
}

hipError_t launch_bwd_dkv(const BwdArgs &a_in, bool causal, bool dropout, hipStream_t st) {
    BwdArgs a = a_in;
    const int nkblk = (a.S + KP_KWG - 1) / KP_KWG;
    // Key-block pairs (causal, no dropout) give every workgroup the same work,
    // head after head per XCD.  That pays only when each XCD's share fills
    // whole rounds of its 2*CUs/8 workgroup slots; otherwise the single
    // blocks, heaviest first, pack the rounds better.
    const int64_t bh = (int64_t)a.B * a.H, per_xcd = (nkblk + 1) / 2 * (bh / 8);
    const int64_t xcd_slots = 2 * (int64_t)device_cus() / 8;
    a.dkv_pair = causal && !dropout && bh % 8 == 0 && per_xcd > 0 && per_xcd % xcd_slots == 0;
    const int nwg = a.dkv_pair ? (nkblk + 1) / 2 : nkblk;
    const dim3 grid((unsigned)(nwg * a.B * a.H)), block(256);
    // The folded row terms need -lse2/scale2 finite (|lse2| < 3e18 at this bound).
    const bool fold = !dropout && a.scale2 >= 1e-20f;
    const bool dmask = dropout && a.drop_mask != nullptr;
    if (causal) {
        if (dmask)
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<true, true, false, true>), grid, block, 0, st, a);
        else if (dropout)
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<true, true, false, false>), grid, block, 0, st, a);
        else if (fold)
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<true, false, true, false>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<true, false, false, false>), grid, block, 0, st, a);
    } else {
        if (dmask)
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<false, true, false, true>), grid, block, 0, st, a);
        else if (dropout)
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<false, true, false, false>), grid, block, 0, st, a);
        else if (fold)
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<false, false, true, false>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((bwd_dkv_pipe_kernel<false, false, false, false>), grid, block, 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace fa2
