// fa2_fwd.hip -- causal FlashAttention-2 forward for gfx950 (MI355X).
//
// Computes, per (b, h) and query row i,
//   O[i]   = sum_j softmax_j(scale * q_i . k_j, j visible) * keep_ij/(1-p) * v_j
//   LSE[i] = ln sum_{j visible} exp(scale * q_i . k_j)
// following the reference's algorithm and guards (reference @ None:
// csrc/flash_attn_v100/flash_attn_v100.cu:109-308): online softmax over key
// tiles, causal tiles past the diagonal skipped, the denominator summed from
// the un-dropped P, O = acc / l with l == 0 -> 0, LSE in natural log.
//
// Work decomposition (one workgroup = 4 waves of one (b, h)); three loops,
// chosen per call by launch_fwd_t:
//   * NARROW (the training shapes, with or without dropout and keep-bit
//     words, and large prefill chunks): each wave owns one 32-query block,
//     the tile loop runs in order (scores, softmax, P V) with two LDS stages
//     (one tile read, one in flight) and one barrier per tile, and at most
//     128 registers per lane let four workgroups share a CU: the other three
//     waves of the SIMD cover a wave's latencies;
//   * two query blocks per wave (smaller grids that still fill two
//     workgroups per CU, without keep-bit words): every K and V operand
//     fragment read from LDS feeds the MFMAs of both blocks, the tile loop
//     runs in order with four stages (one read, three in flight);
//   * one query block per wave, software pipelined (short query ranges,
//     key slices): step t issues the P V MFMAs of tile t-1 and the score
//     MFMAs of tile t+1 while the VALU forms P of tile t, in chunks that pair
//     two MFMAs with four exponentials; four stages (three resident, one in
//     flight);
//   * a wave's Q^T operands (16 x 32 fp16 per d-step and block) stay in
//     registers for the whole kernel;
//   * key tiles of 64 keys are moved global -> LDS by the waves' direct
//     transfers (global_load_lds, no register staging; a scalar tile base
//     plus fixed 32-bit lane offsets) into XOR-swizzled tiles; K feeds the A
//     operand of S^T = K Q^T with 16-byte reads, V feeds the A operand of
//     O^T = V^T P^T through transposing ds_read_b64_tr_b16 reads, both free
//     of LDS bank conflicts;
//   * S^T accumulators give each lane one query and 32 keys, so the row max
//     is a local max plus one cross-half exchange, the running sum l stays a
//     per-lane partial until the epilogue, the O^T rescale is a per-lane
//     scalar, and P goes from the accumulator straight into the B operand of
//     the PV MFMA (no LDS round trip);
//   * no per-tile row max: P is formed against a lazily updated reference
//     max and an overflow check on its row sum (v_dot2_f32_f16 on the packed
//     fp16 P) decides when the true max, the O/l rescale and a recompute are
//     needed, which is almost never after the first tile;
//   * workgroups are issued heaviest first (last query blocks first) and all
//     workgroups of one (b, h) share blockIdx % 8, i.e. one XCD and its L2.
#include "fa2_device.h"
#include "fa2_kernels.h"

namespace fa2 {
namespace {

#ifndef FA2_FWD_NW
#define FA2_FWD_NW 4
#endif
constexpr int NW = FA2_FWD_NW;     // waves per workgroup (4 or 8)
constexpr int TPW = 8 / NW;        // 1 KB tile transfers per wave and tensor
constexpr int KT = 64;             // keys per tile
// 32-query blocks per wave (template parameter QBT of fwd_kernel):
//   1: the software-pipelined step below (two tiles' matrix work beside one
//      tile's softmax in every wave);
//   2: each K / V operand fragment read from LDS feeds both query blocks, and
//      the tile loop is not pipelined inside the wave (scores, softmax, PV in
//      order): the other wave on the SIMD overlaps it.
constexpr int qwg_of(int qbt) { return NW * 32 * qbt; }   // queries per workgroup
#ifndef FA2_FWD_NST
#define FA2_FWD_NST 4
#endif
constexpr int NST = FA2_FWD_NST;   // LDS stages of (K, V) tiles: 4 or 5
constexpr float P_SUM_LIMIT = 32768.f;  // per-lane partial sum bound: every P <= 2^15

// SPLIT: the key range is cut into a.nsplit slices of a.split_keys keys; the
// workgroup of slice ks runs the same pipeline over its slice and writes the
// unnormalised partial result (O accumulator, reference max, row sum) for
// fwd_combine_kernel instead of O and LSE.
//
// DMASK (dropout, no key slices): each lane also stores its tile's 32 keep
// bits as one word of a.drop_mask (dmask_word layout), for the backward.
//
// NARROW (one query block per wave): the in-order loop with one barrier per
// tile and, by default (NARROW_WAVES = 4), two LDS stages and at most 128
// registers per lane, so that four workgroups (four waves per SIMD) share a
// CU; NARROW_WAVES = 3 gives three stages and 168 registers.  With one query
// block a wave's scores -> softmax -> P V chain is short, and the other waves
// of the SIMD cover its latencies.
#ifndef FA2_FWD_NARROW_WAVES
#define FA2_FWD_NARROW_WAVES 4
#endif
constexpr int NARROW_WAVES = FA2_FWD_NARROW_WAVES;   // waves per SIMD of the narrow loop: 3 or 4
static_assert(NARROW_WAVES == 3 || NARROW_WAVES == 4, "three or four narrow waves per SIMD");

template <bool CAUSAL, bool DROPOUT, bool SPLIT, bool DMASK, int QBT, bool NARROW = false>
__global__ __launch_bounds__(NW * 64, NARROW ? NARROW_WAVES : 8 / NW) void fwd_kernel(const FwdArgs a) {
    constexpr int QB = QBT;
    constexpr int QWG = qwg_of(QBT);
    constexpr bool NOPIPE = QBT == 2 || NARROW;
    // LDS stages of this variant (narrow: 48 KB or 32 KB per workgroup, so
    // that three or four workgroups fit the CU's 160 KB).
    constexpr int NSK = NARROW ? (NARROW_WAVES == 4 ? 2 : 3) : NST;
    static_assert(QBT == 1 || QBT == 2, "one or two query blocks per wave");
    static_assert(!NARROW || QBT == 1, "the narrow loop holds one query block per wave");
    static_assert(!DMASK || (DROPOUT && !SPLIT && (NARROW || NST == 4)), "keep-bit words: the unsplit forward");
    static_assert(!(DMASK && QBT == 2), "keep-bit words: the one-block loops");
    static_assert(!NOPIPE || NARROW || NST == 4, "the unpipelined loop's waits assume four stages");
    // NSK stages of one K tile and one V tile (8 KB each, swizzled chunks).
    __shared__ __attribute__((aligned(16))) h8 sKV[NSK][2][KT * 8];
    // Dropout: per wave, the column part dropout_xs16(col term) of the
    // current tile's KT keys, formed once per key and read by every lane.
    __shared__ __attribute__((aligned(16))) uint32_t sDK[DROPOUT ? NW * KT : 1];
    // NARROW: each lane's four transfer offsets of a full tile (K rows i = 0,
    // 1, then V rows), 1 KB per wave.
    typedef uint32_t u4x __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) u4x sOff[NARROW ? NW * 64 : 1];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar
    const int lane = tid & 63, c = lane & 31, g2 = lane >> 5;
    const int S = a.S;       // query rows
    const int Sk = a.Sk;     // key rows
    const int coff = a.coff; // causal: key j visible to query i iff j <= i + coff
    const int BH = a.B * a.H;
    const int nqblk = (S + QWG - 1) / QWG;
    const int nsplit = SPLIT ? a.nsplit : 1;
    const int L = blockIdx.x;
    // Split: (query slot, slice, b*H + h), heads fastest; otherwise
    // query_block_order (heaviest query blocks first, a head on one XCD).
    int qslot, ks = 0, bh;
    if (SPLIT) {
        qslot = L / (BH * nsplit);
        const int rem = L - qslot * (BH * nsplit);
        ks = rem / BH;
        bh = rem - ks * BH;
    } else {
        query_block_order(L, BH, nqblk, a.hgroup, qslot, bh);
    }
    const int qblk = nqblk - 1 - qslot;                // heaviest (last) query blocks first
    const int b = bh / a.H, h = bh - b * a.H;

    const _Float16 *Qp = a.q + b * a.qsb + h * a.qsh;
    const _Float16 *Kp = a.k + b * a.ksb + h * a.ksh;
    const _Float16 *Vp = a.v + b * a.vsb + h * a.vsh;
    _Float16 *Op = a.o + b * a.osb + h * a.osh;
    float *Lp = a.lse + b * a.lsb + h * a.lsh;

    const int q_wg0 = qblk * QWG;
    const int qw0 = q_wg0 + wave * 32 * QB;   // this wave's queries: qw0 .. qw0 + 32*QB - 1
    const float scale2 = a.scale2;

    // Keys kbase .. kend-1, in tiles t = 0 .. ntiles-1 starting at key kbase.
    const int kbase = SPLIT ? ks * a.split_keys : 0;   // split_keys: a multiple of KT
    const int kend_wg = CAUSAL ? min(Sk, q_wg0 + QWG + coff) : Sk;
    const int kend = SPLIT ? min(kend_wg, kbase + a.split_keys) : kend_wg;
    const int ntiles = kend > kbase ? (kend - kbase + KT - 1) / KT : 0;
    // Last key tile this wave computes (-1: none).  Every wave still joins
    // every barrier and moves its share of every tile.
    const int kw_end = min(CAUSAL ? min(qw0 + 32 * QB + coff, Sk) : Sk, kend);   // keys the wave's queries reach
    const int tlast = (qw0 >= S || kw_end <= kbase) ? -1 : (kw_end - 1 - kbase) / KT;
    // Tiles before tsteady are visible to every query of the wave (the
    // steady, mask-free path); the rest run the general path.
    const int tsteady = CAUSAL ? min(tlast, max(qw0 + coff + 1 - kbase, 0) / KT) : tlast;

    // Q^T operand of d-step st: lane holds Q[q][16*st + 8*g2 + e].  Rows past
    // S load row S - 1 (unconditional loads stay in flight together); those
    // lanes' results are never stored.  Loaded before the first tiles, so
    // waiting for a tile also covers them.
    h8 qf[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const _Float16 *qrow = Qp + (int64_t)min(qw0 + 32 * qb + c, S - 1) * a.qss + 8 * g2;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const h8 v = *reinterpret_cast<const h8 *>(qrow + 16 * st);
            qf[qb][st] = neg_h8_if(v, a.negate);
        }
    }

    // Tile loader: the 512 16-byte chunks of a K (or V) tile are 8 transfers
    // of 64 lanes; wave w moves transfers j = 2w, 2w+1 of both.  Lane L of
    // transfer j lands at chunk position 64j + L = 8*row + (L & 7) with
    // row = 8j + (L >> 3), so it fetches logical chunk (L & 7) ^ swz(row) of
    // key row k0 + row.  The lane's byte offsets within a tile are fixed; only
    // the last tile, whose rows past Sk are redirected to row Sk - 1 (any
    // finite row: their scores are masked and their P is zero), needs them
    // recomputed.  The narrow variant, whose four waves per SIMD leave no
    // registers to hold them across the tile loop, keeps them in an LDS slot
    // of the wave and reads them back with one ds_read_b128 per tile (its
    // last, partial tile recomputes them from the lane index, re-read through
    // an opaque move so that nothing derived from it stays live across the
    // loop).  Recomputing every tile cost ~25 VALU instructions per tile.
    auto tile_offsets = [&](int k0, uint32_t(&ko)[2], uint32_t(&vo)[2]) FA2_INLINE {
        int ln = lane;
        if (NARROW) asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
        const int lrow = ln >> 3;
        const int kch[2] = {(ln & 7) ^ swz_rows(lrow), (ln & 7) ^ swz_rows(lrow + 8)};
        const int vch = (ln & 7) ^ swz_tr(lrow);
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int row = min(k0 + 8 * (TPW * wave + i) + lrow, Sk - 1) - k0;
            ko[i] = (mul_u24((uint32_t)a.kss, (uint32_t)row) + 8 * kch[(TPW * wave + i) & 1]) * 2u;   // kss < 2^24 (host check)
            vo[i] = (mul_u24((uint32_t)a.vss, (uint32_t)row) + 8 * vch) * 2u;
        }
    };
    // Stage of tile t (t >= 0; unsigned, so a power-of-two count is a mask).
    auto stage_of = [](int t) FA2_INLINE { return (int)((uint32_t)t % (uint32_t)NSK); };
    uint32_t koffg[2] = {0u, 0u}, voffg[2] = {0u, 0u};
    if (!NARROW) {
        tile_offsets(0, koffg, voffg);
    } else {
        // A full tile's offsets (with Sk < KT every tile is partial and
        // recomputes them, so the clamped values stored then go unread).
        uint32_t ko[2], vo[2];
        tile_offsets(0, ko, vo);
        sOff[64 * wave + lane] = u4x{ko[0], ko[1], vo[0], vo[1]};
    }
    // Tiles are issued in order, once each: issue_next() sends the next tile
    // (the callers' index tests only decide whether there is one).  Scalar
    // running addresses (global tile bases, LDS stage) advance by a constant
    // per tile instead of being recomputed with 64-bit multiplies at every
    // transfer.
    uint64_t gk = (uint64_t)(uintptr_t)(Kp + (int64_t)kbase * a.kss);
    uint64_t gv = (uint64_t)(uintptr_t)(Vp + (int64_t)kbase * a.vss);
    const uint64_t k_step = (uint64_t)KT * a.kss * 2, v_step = (uint64_t)KT * a.vss * 2;
    int kn = kbase;      // first key of the next tile to issue
    uint32_t stn = 0;    // its stage
    const uint32_t lds_kv = lds_addr(&sKV[0][0][0]) + 1024u * (uint32_t)(TPW * wave);
    auto issue_next = [&]() FA2_INLINE {
        uint32_t ko[2] = {koffg[0], koffg[1]}, vo[2] = {voffg[0], voffg[1]};
        if (kn + KT > Sk) {
            tile_offsets(kn, ko, vo);
        } else if (NARROW) {
            // An opaque slot address: the read stays in the loop instead of
            // being hoisted into four live registers.  With keep-bit words
            // it is formed from an opaque copy of the lane index every tile,
            // so that no register holds it across the loop (kept live, that
            // variant spilled it to scratch and reloaded it at every tile).
            uint32_t oa;
            if (DMASK) {
                uint32_t ln;
                asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
                oa = lds_addr(&sOff[64 * wave]) + 16u * ln;
            } else {
                oa = lds_addr(&sOff[64 * wave]) + 16u * (uint32_t)lane;
                asm volatile("" : "+v"(oa));
            }
            const u4x ov = *reinterpret_cast<const __attribute__((address_space(3))) u4x *>(oa);
            ko[0] = ov[0];
            ko[1] = ov[1];
            vo[0] = ov[2];
            vo[1] = ov[3];
        }
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const uint32_t d = lds_kv + stn * (uint32_t)sizeof(sKV[0]) + 1024u * (uint32_t)i;
            lds_dma16_at(gk, ko[i], d);
            lds_dma16_at(gv, vo[i], d + (uint32_t)sizeof(sKV[0][0]));
        }
        gk += k_step;
        gv += v_step;
        kn += KT;
        stn = (stn + 1 == NSK) ? 0 : stn + 1;
    };
#pragma unroll
    for (int t = 0; t < NSK - 1; ++t)
        if (t < ntiles) issue_next();

    f16x o[QB][2];                      // O^T, d blocks 0..31 and 32..63
    float msc[QB], l[QB];               // reference max (log2 units), per-lane partial row sum
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        o[qb][0] = zero16();
        o[qb][1] = zero16();
        msc[qb] = -INFINITY;
        l[qb] = 0.f;
    }

    // Per-lane LDS byte offsets of the operand reads.
    //   K (A operand of S^T): row c (+32 for kb = 1), logical chunk 2*st + g2.
    int koff[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) koff[st] = c * 128 + (((2 * st + g2) ^ swz_rows(c)) << 4);
    //   V^T (A operand of O^T, transposing reads), d block db.
    const int voff0 = tr_lane_off(0), voff1 = tr_lane_off(32);

    auto kread = [&](int stage, int st, int kb) FA2_INLINE {
        return *reinterpret_cast<const h8 *>(reinterpret_cast<const char *>(sKV[stage][0]) + koff[st] +
                                              kb * 32 * 128);
    };
    auto vread = [&](int stage, int db, int kb, int hh) FA2_INLINE {
        return tr_read8_sw(reinterpret_cast<const _Float16 *>(sKV[stage][1]), db ? voff1 : voff0,
                           32 * kb + 16 * hh);
    };
    // S^T = K Q^T against the K tile in `stage`: s[kb] rows = keys
    // 32*kb + (8i+4g2+j) of the tile, column = this lane's query.  The reads
    // run one d-step ahead; the scheduling barriers keep the compiler from
    // hoisting all of them, which would raise the kernel's register peak.
    auto s_mm = [&](int stage, f16x(&s)[QB][2]) FA2_INLINE {
        h8 n0 = kread(stage, 0, 0), n1 = kread(stage, 0, 1);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const h8 f0 = n0, f1 = n1;
            if (st < 3) {
                n0 = kread(stage, st + 1, 0);
                n1 = kread(stage, st + 1, 1);
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if (st == 0) {   // C = inline constant 0
                    s[qb][0] = mfma32_first(f0, qf[qb][0]);
                    s[qb][1] = mfma32_first(f1, qf[qb][0]);
                } else {
                    s[qb][0] = mfma32(f0, qf[qb][st], s[qb][0]);
                    s[qb][1] = mfma32(f1, qf[qb][st], s[qb][1]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // O^T += V^T P^T over the V tile in `stage`, 16 keys per MFMA.
    auto pv = [&](int stage, const h8(&pb)[QB][2][2]) FA2_INLINE {
        h8 n0 = vread(stage, 0, 0, 0), n1 = vread(stage, 1, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {   // (kb, hh) = (i >> 1, i & 1)
            const h8 f0 = n0, f1 = n1;
            if (i < 3) {
                n0 = vread(stage, 0, (i + 1) >> 1, (i + 1) & 1);
                n1 = vread(stage, 1, (i + 1) >> 1, (i + 1) & 1);
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                o[qb][0] = mfma32(f0, pb[qb][i >> 1][i & 1], o[qb][0]);
                o[qb][1] = mfma32(f1, pb[qb][i >> 1][i & 1], o[qb][1]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Tail keys (>= Sk) and the causal triangle -> -inf.  key = k0 + 32*kb +
    // 4*g2 + (8*(r>>2) + (r&3)) is visible iff key <= lim; compared as a
    // constant against a per-lane bound, so no key index is materialised.
    auto need_mask = [&](int k0) FA2_INLINE {
        return (k0 + KT > Sk) || (CAUSAL && k0 + KT - 1 > qw0 + coff);
    };
    auto mask = [&](int qb, int k0, f16x(&s)[2]) FA2_INLINE {
        const int lim = CAUSAL ? min(qw0 + 32 * qb + c + coff, Sk - 1) : Sk - 1;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int bound = lim - k0 - 32 * kb - 4 * g2;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (8 * (r >> 2) + (r & 3) > bound) s[kb][r] = -INFINITY;
        }
    };
    // Online softmax against a lazily updated reference max msc (log2 units).
    // P = exp2(s*scale2 - msc) is formed straight away, without a row max:
    // the lane's fp16 P values are summed (fp32, v_dot2), and a partial sum
    // <= 2^15 proves no P overflowed fp16.  Only when a sum exceeds that (or
    // is inf/NaN, as on the first tile where msc = -inf) does the cold path
    // take the true row max, rescale O and l, and form P again.  l and LSE
    // use whatever msc is current, so the result is the exact online softmax;
    // the reference max only bounds the magnitudes (P <= 2^15).
    // The lane's partial row sum is kept as four sums, one per (kb, hh) group
    // of eight elements, added pairwise at the end: four short dependency
    // chains of v_dot2 instead of one of sixteen.  (The pipelined step sums
    // the same elements in the same order, so both loops give the same bits.)
    auto p_form = [&](const f16x(&s)[2], float sub, h8(&pb)[2][2]) FA2_INLINE {
        float part[4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                f8 x;
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * hh + e], scale2, -sub));
                pb[kb][hh] = __builtin_convertvector(x, h8);
                part[2 * kb + hh] = sum_h8(pb[kb][hh], 0.f);
            }
        return (part[0] + part[1]) + (part[2] + part[3]);
    };
    // After P of tile k0 (K tile in `stage`) was formed with partial sum rs:
    // the cold path (scores recomputed from the K tile, so no score register
    // has to outlive P), dropout, and the running sum.
    uint32_t wpend = 0;   // DMASK: the keep word of the tile being finished
    // Dropout on the P of query block qb, tile k0 (l already holds its
    // un-dropped sum); returns the keep word (DMASK) of the lane's query.
    auto drop_apply = [&](int qb, int k0, h8(&pb)[2][2]) FA2_INLINE -> uint32_t {
        // l sums the un-dropped P; dropout then zeroes the dropped elements
        // of P in place (the 1/(1-p) of the kept ones scales O once, in the
        // epilogue).  The hash of element (query, key) is the finaliser of
        // row part ^ column term, taken apart as dropout_xs16 of each part
        // (the column parts of the tile's 64 keys one per lane, through this
        // wave's LDS slot: the wave's own stores precede its reads, in
        // order) and dropout_mix_tail, compared with T = thr << 8.  Per
        // element: the compare into VCC, then an SDWA v_cndmask that
        // rewrites the element's 16-bit half of the packed pair with itself
        // or 0 and preserves the other half.  DMASK: the same VCC bit enters
        // the word by v_addc_co (w = 2w + keep), so element 16*kb + 8*hh + e
        // lands on bit 31 - (16*kb + 8*hh + e).
        uint32_t *const kpart = &sDK[DROPOUT ? KT * wave : 0];
        kpart[lane] = dropout_xs16(dropout_col_term(k0 + lane));
        uint32_t w = 0;
        const uint32_t hthr = a.drop_thr << 8, thi = hthr >> 16;
        const uint32_t rpart = dropout_xs16(dropout_row_part(a.seed, qw0 + 32 * qb + c, (uint32_t)bh));
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                typedef uint32_t u4x __attribute__((ext_vector_type(4)));
                u4x pk = __builtin_bit_cast(u4x, pb[kb][hh]);
                // keys 32*kb + 16*hh + 8*m + 4*g2 + (0..3) of the tile
                const u4x kp0 = *reinterpret_cast<const u4x *>(&kpart[32 * kb + 16 * hh + 4 * g2]);
                const u4x kp1 = *reinterpret_cast<const u4x *>(&kpart[32 * kb + 16 * hh + 8 + 4 * g2]);
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    uint32_t r = pk[e2];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int e = 2 * e2 + j;   // key 8*(e >> 2) + 4*g2 + (e & 3) of the 16
                        const uint32_t h = dropout_mix_tail(rpart ^ ((e >> 2) ? kp1[e & 3] : kp0[e & 3]), thi);
                        if (j == 0 && DMASK)
                            asm("v_cmp_le_u32 vcc, %3, %2\n\t"
                                "v_cndmask_b32_sdwa %0, 0, %0, vcc dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE "
                                "src0_sel:WORD_0 src1_sel:WORD_0\n\t"
                                "v_addc_co_u32 %1, vcc, %1, %1, vcc"
                                : "+v"(r), "+v"(w) : "v"(h), "s"(hthr) : "vcc");
                        else if (DMASK)
                            asm("v_cmp_le_u32 vcc, %3, %2\n\t"
                                "v_cndmask_b32_sdwa %0, 0, %0, vcc dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE "
                                "src0_sel:WORD_1 src1_sel:WORD_1\n\t"
                                "v_addc_co_u32 %1, vcc, %1, %1, vcc"
                                : "+v"(r), "+v"(w) : "v"(h), "s"(hthr) : "vcc");
                        else if (j == 0)
                            asm("v_cmp_le_u32 vcc, %2, %1\n\t"
                                "v_cndmask_b32_sdwa %0, 0, %0, vcc dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE "
                                "src0_sel:WORD_0 src1_sel:WORD_0"
                                : "+v"(r) : "v"(h), "s"(hthr) : "vcc");
                        else
                            asm("v_cmp_le_u32 vcc, %2, %1\n\t"
                                "v_cndmask_b32_sdwa %0, 0, %0, vcc dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE "
                                "src0_sel:WORD_1 src1_sel:WORD_1"
                                : "+v"(r) : "v"(h), "s"(hthr) : "vcc");
                    }
                    pk[e2] = r;
                }
                pb[kb][hh] = __builtin_bit_cast(h8, pk);
            }
        return w;
    };
    auto softmax_tail = [&](int qb, int k0, int stage, h8(&pb)[2][2], float rs) FA2_INLINE {
        if (__any(!(rs <= P_SUM_LIMIT))) {
            FA2_COLD_BRANCH();
            f16x sq[QB][2];
            s_mm(stage, sq);
            f16x(&s)[2] = sq[qb];
            if (need_mask(k0)) mask(qb, k0, s);
            float mx = s[0][0];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
            mx = fmaxf(mx, xor32(mx));
            const float mnew = fmaxf(msc[qb], mx * scale2);
            // mnew == -inf: every key so far masked; alpha stays 1 with O, l = 0
            const float alpha = (mnew == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(msc[qb] - mnew);
            msc[qb] = mnew;
            l[qb] *= alpha;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[qb][db][r] *= alpha;
            rs = p_form(s, (mnew == -INFINITY) ? 0.f : mnew, pb);
        }
        if (DROPOUT) {
            const uint32_t w = drop_apply(qb, k0, pb);
            if (DMASK) wpend = w;   // stored by tile_end
        }
        l[qb] += rs;
    };
    // Steady-state step: O^T += V^T P_prev^T from V stage sv, s_next = K Q^T
    // from K stage sk, and P_cur = exp2(s_cur * scale2 - msc), returning the
    // lane's partial sum of P_cur.  Eight chunks, each two MFMAs and four
    // exponentials, separated by scheduling barriers, with the operand reads
    // of chunk i+1 issued in chunk i.  The PV MFMAs come first, while the
    // first half of s_cur is consumed, and the score MFMAs second, so s_next
    // only occupies registers once P_prev and half of s_cur are dead.
    auto step = [&](int sk, int sv, f16x(&s_next)[QB][2], const h8(&p_prev)[QB][2][2], const f16x(&s_cur)[QB][2],
                    h8(&p_cur)[QB][2][2], float(&rs)[QB]) FA2_INLINE {
        // chunk i < 4: PV for (kb, hh) = (i >> 1, i & 1), d blocks 0 and 1;
        // chunk i >= 4: scores for d-step i - 4, key blocks 0 and 1; each for
        // every query block, with the operand fragments shared.
        h8 n0 = vread(sv, 0, 0, 0), n1 = vread(sv, 1, 0, 0);
        float part[QB][4];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int j = 0; j < 4; ++j) part[qb][j] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const h8 f0 = n0, f1 = n1;
            if (i < 3) {
                n0 = vread(sv, 0, (i + 1) >> 1, (i + 1) & 1);
                n1 = vread(sv, 1, (i + 1) >> 1, (i + 1) & 1);
            } else if (i < 7) {
                n0 = kread(sk, i - 3, 0);
                n1 = kread(sk, i - 3, 1);
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if (i < 4) {
                    o[qb][0] = mfma32(f0, p_prev[qb][i >> 1][i & 1], o[qb][0]);
                    o[qb][1] = mfma32(f1, p_prev[qb][i >> 1][i & 1], o[qb][1]);
                } else if (i == 4) {
                    s_next[qb][0] = mfma32_first(f0, qf[qb][0]);
                    s_next[qb][1] = mfma32_first(f1, qf[qb][0]);
                } else {
                    s_next[qb][0] = mfma32(f0, qf[qb][i - 4], s_next[qb][0]);
                    s_next[qb][1] = mfma32(f1, qf[qb][i - 4], s_next[qb][1]);
                }
                // elements 4i .. 4i+3 of s_cur: kb = i >> 2, hh = (i >> 1) & 1, e0 = 4 (i & 1)
                const int kb2 = i >> 2, hh2 = (i >> 1) & 1, e0 = 4 * (i & 1);
                f4 x;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    x[e] = __builtin_amdgcn_exp2f(fmaf(s_cur[qb][kb2][8 * hh2 + e0 + e], scale2, -msc[qb]));
                const h4 ph = __builtin_convertvector(x, h4);
#pragma unroll
                for (int e = 0; e < 4; ++e) p_cur[qb][kb2][hh2][e0 + e] = ph[e];
                const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
                float &pj = part[qb][i >> 1];   // group (kb2, hh2)
                pj = __builtin_amdgcn_fdot2(__builtin_shufflevector(ph, ph, 0, 1), one, pj, false);
                pj = __builtin_amdgcn_fdot2(__builtin_shufflevector(ph, ph, 2, 3), one, pj, false);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) rs[qb] = (part[qb][0] + part[qb][1]) + (part[qb][2] + part[qb][3]);
    };

    // Software pipeline over key tiles:
    //   step t: PV(t-1) with V_{t-1} | S(t+1) = K_{t+1} Q^T | P(t) from S(t)
    // then the cold path of P(t) (which may re-read K_t), then one barrier.
    // Tiles t-1 .. t+1 are resident during step t and tiles t+2 .. t+NST-2
    // are in flight.  The barrier after step t publishes tile t+2 and frees
    // the stage of tile t-1 for tile t+NST-1.
    static_assert(NST == 4 || NST == 5, "three resident tiles plus one or two in flight");
    // One tile of the in-order loops: scores, masking, softmax (with its cold
    // path on the live scores), dropout, P V; returns the keep word of query
    // block 0 (DMASK).
    auto inorder_tile = [&](int t, int stage, f16x(&s)[QB][2], h8(&p)[QB][2][2]) FA2_INLINE -> uint32_t {
        const int k0 = kbase + t * KT;
        uint32_t w = 0;
        s_mm(stage, s);
        if (need_mask(k0)) {
            FA2_COLD_BRANCH();
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) mask(qb, k0, s[qb]);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            float rs;
            if (!DMASK && t == 0) {
                // First tile: msc is -inf, so P against it would only fail
                // the overflow check into the cold path (a second P pass).
                // Take the row max from the live scores directly, as the
                // cold path would (with O and l still zero its rescale is a
                // no-op), so the result is the same bits; -inf when every key
                // is masked.  (With keep-bit words this copy would spill;
                // they keep the cold path, with the same result.)
                float mx = s[qb][0][0];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][kb][r]);
                mx = fmaxf(mx, xor32(mx)) * scale2;
                msc[qb] = mx;
                rs = p_form(s[qb], (mx == -INFINITY) ? 0.f : mx, p[qb]);
            } else {
                rs = p_form(s[qb], msc[qb], p[qb]);
            }
            if (__any(!(rs <= P_SUM_LIMIT))) {
                // The cold path on the live scores: true row max, rescale of
                // O and l, P again (almost never after the first tile).
                FA2_COLD_BRANCH();
                float mx = s[qb][0][0];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][kb][r]);
                mx = fmaxf(mx, xor32(mx));
                const float mnew = fmaxf(msc[qb], mx * scale2);
                const float alpha = (mnew == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(msc[qb] - mnew);
                msc[qb] = mnew;
                l[qb] *= alpha;
#pragma unroll
                for (int db = 0; db < 2; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[qb][db][r] *= alpha;
                rs = p_form(s[qb], (mnew == -INFINITY) ? 0.f : mnew, p[qb]);
            }
            l[qb] += rs;
            if (DROPOUT) {
                const uint32_t wq = drop_apply(qb, k0, p[qb]);
                if (qb == 0) w = wq;
            }
        }
        pv(stage, p);
        return w;
    };
    if constexpr (NARROW) {
        // NSK stages: tile t is read while tiles t+1 .. t+NSK-1 are in
        // flight.  The end of tile t waits for tile t+1 (the transfers of
        // tiles t+2 .. t+NSK-1 may still be pending), joins the barrier
        // after which no wave reads stage t % NSK any more, and sends tile
        // t+NSK there.  DMASK: the tile's keep word is stored after that
        // wait; a store still in flight at the next wait only makes its count
        // stricter (the loads complete in order), so the waits stay exact.
        auto wait_tiles = [&](int n) FA2_INLINE {   // at most n tiles' transfers pending
            if (n <= 0) vm_wait<0>();
            else if (n == 1) vm_wait<2 * TPW>();
            else vm_wait<4 * TPW>();
        };
#ifndef FA2_FWD_STORE_SLACK
#define FA2_FWD_STORE_SLACK 0
#endif
        // The same with the previous tile's keep-word store (issued after
        // every transfer being waited for) allowed to stay in flight.
        auto wait_tiles_st = [&](int n) FA2_INLINE {
            if (n <= 0) vm_wait<1>();
            else if (n == 1) vm_wait<2 * TPW + 1>();
            else vm_wait<4 * TPW + 1>();
        };
        if (NSK - 1 < ntiles) issue_next();   // the last stage's tile (the prologue sent the others)
        wait_tiles(min(NSK - 1, ntiles - 1));
        lds_barrier();                         // tile 0 landed for every wave
        f16x s[QB][2];
        h8 p[QB][2][2];
        // Unrolled over the NSK stages (tile t sits in stage t % NSK, and
        // every wave starts at tile 0), so that each copy's stage is a
        // constant and the operand reads address LDS through instruction
        // offsets, with no per-tile address arithmetic.  (With keep-bit
        // words the copies would spill: one copy, the stage at run time.)
        constexpr int U = DMASK ? 1 : NSK;
        for (int t0 = 0; t0 < ntiles; t0 += U) {
#pragma unroll
            for (int ph = 0; ph < U; ++ph) {
                const int t = t0 + ph;
                if (t >= ntiles) break;
                uint32_t w = 0;
                if (t <= tlast) w = inorder_tile(t, U == 1 ? stage_of(t) : ph, s, p);
                if (t + 1 < ntiles) {
                    if (DMASK && FA2_FWD_STORE_SLACK && t >= 1 && t - 1 <= tlast)
                        wait_tiles_st(min(NSK - 2, ntiles - 2 - t));
                    else
                        wait_tiles(min(NSK - 2, ntiles - 2 - t));   // tile t+1 landed
                    lds_barrier();
                    if (t + NSK < ntiles) issue_next();
                }
                if (DMASK && t <= tlast) {
                    const int q = qw0 + c;   // QB == 1
                    if (q < S) a.drop_mask[dmask_word(CAUSAL, bh, S, kbase / KT + t, g2, q)] = w;
                }
            }
        }
        vm_wait<0>();
        lds_barrier();   // every wave is done with the stages: the epilogue reuses them
    } else if constexpr (NOPIPE) {
        // Tiles are computed in pairs with one barrier after each pair: while
        // tiles t-1, t are read, t+1, t+2 are in flight; the pair's end waits
        // for those two (every issued transfer) and refills the two stages
        // just read with tiles t+3, t+4.  Tile 3 goes out now.
        if (NST - 1 < ntiles) issue_next();
        auto wait_pending = [&](int n) FA2_INLINE {   // at most n tiles' transfers in flight
            if (n <= 0) vm_wait<0>();
            else if (n == 1) vm_wait<2 * TPW>();
            else if (n == 2) vm_wait<4 * TPW>();
            else vm_wait<6 * TPW>();
        };
        wait_pending(min(NST - 2, ntiles - 2));   // tiles 0 and 1 landed
        lds_barrier();
        f16x s[QB][2];
        h8 p[QB][2][2];
        for (int t = 0; t < ntiles; ++t) {
            if (t <= tlast) (void)inorder_tile(t, stage_of(t), s, p);
            if (!(t & 1) && t + 1 < ntiles) continue;   // the pair's first tile
            vm_wait<0>();                                // tiles t+1, t+2 (the next pair) landed
            lds_barrier();                               // every wave is done with tiles t-1, t
            if (t + 3 < ntiles) issue_next();
            if (t + 4 < ntiles) issue_next();
        }
    } else {
    // Tiles 0 and 1 have landed once at most the transfers of tiles
    // 2 .. NST-2 are pending (4 per tile and wave).
    if (NST == 5 && ntiles >= 4) vm_wait<8>(); else if (ntiles >= 3) vm_wait<4>(); else vm_wait<0>();
    lds_barrier();

    f16x s0[QB][2], s1[QB][2];          // scores of even / odd tiles
    h8 p0[QB][2][2], p1[QB][2][2];      // P of even / odd tiles
    if (tlast >= 0) s_mm(0, s0);
    // Tile t keeps its scores and P in (s0, p0) for even t and (s1, p1) for
    // odd t.  The end of a tile: tile t+2 landed (tiles up to t+NST-2 are
    // issued), the barrier, and tile t+NST-1 into the stage of tile t-1.
    // DMASK: a computed tile's (t <= tlast) keep word is stored here, after
    // the wait, the barrier and the next tile's transfers, so the count-based
    // wait stays vmcnt(0) -- it needs no ordering between loads and stores --
    // and the store has a whole step to complete before the next one.
    auto tile_end = [&](int t) FA2_INLINE {
        if (NST == 5 && t + 3 < ntiles) vm_wait<4>();
        else if (t + 2 < ntiles) vm_wait<0>();
        lds_barrier();
        if (t + NST - 1 < ntiles) issue_next();
        if (DMASK && t <= tlast) {
            const int q = qw0 + c;   // QB == 1
            if (q < S) a.drop_mask[dmask_word(CAUSAL, bh, S, kbase / KT + t, g2, q)] = wpend;
        }
    };
    // Steady state (1 <= t < tsteady): no masking -- the tile is below this
    // wave's diagonal and not the last one -- and every group present.
    auto steady = [&](int t, f16x(&s_cur)[QB][2], h8(&p_cur)[QB][2][2], f16x(&s_nxt)[QB][2],
                      h8(&p_prv)[QB][2][2]) FA2_INLINE {
        float rs[QB];
        step(stage_of(t + 1), stage_of(t + NST - 1), s_nxt, p_prv, s_cur, p_cur, rs);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) softmax_tail(qb, kbase + t * KT, stage_of(t), p_cur[qb], rs[qb]);
        tile_end(t);
    };
    // First tile, this wave's last (diagonal / tail) tile, and the tiles after
    // it, where the wave only drains PV and keeps moving its share of tiles.
    auto general = [&](int t, f16x(&s_cur)[QB][2], h8(&p_cur)[QB][2][2], f16x(&s_nxt)[QB][2],
                       h8(&p_prv)[QB][2][2]) FA2_INLINE {
        const int k0 = kbase + t * KT;
        if (t >= 1 && t - 1 <= tlast) pv(stage_of(t + NST - 1), p_prv);
        if (t <= tlast) {
            // Serial order (rare path): each operand dies before the next
            // group's results are born, which keeps the register peak low.
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if (need_mask(k0)) {
                    FA2_COLD_BRANCH();
                    mask(qb, k0, s_cur[qb]);
                }
                float rs;
                if (t == 0) {
                    // First tile: msc is -inf, so P against it would only
                    // overflow into the cold path.  The scores are still
                    // live here: take the row max from them directly (the
                    // value the cold path would compute, -inf when every key
                    // is masked).
                    float mx = s_cur[qb][0][0];
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_cur[qb][kb][r]);
                    mx = fmaxf(mx, xor32(mx)) * scale2;
                    msc[qb] = mx;
                    rs = p_form(s_cur[qb], (mx == -INFINITY) ? 0.f : mx, p_cur[qb]);
                } else {
                    rs = p_form(s_cur[qb], msc[qb], p_cur[qb]);
                }
                softmax_tail(qb, k0, stage_of(t), p_cur[qb], rs);
            }
            if (t + 1 <= tlast) s_mm(stage_of(t + 1), s_nxt);
            if (t == ntiles - 1) pv(stage_of(t), p_cur);   // nothing after it drains P(t)
        }
        tile_end(t);
    };
    // Separate loops keep the steady body free of the general path's code,
    // and every call site has fixed array roles: a role chosen at run time
    // would make the compiler select between whole register arrays.
    if (ntiles > 0) general(0, s0, p0, s1, p1);
    int t = 1;
    for (; t + 1 < tsteady; t += 2) {   // t odd, t + 1 even
        steady(t, s1, p1, s0, p0);
        steady(t + 1, s0, p0, s1, p1);
    }
    if (t < tsteady) {                   // t odd
        steady(t, s1, p1, s0, p0);
        ++t;
    }
    if (t & 1) {
        // Tile t's scores and the previous P move to the even roles, once.
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const f16x ts = s0[qb][kb];
                s0[qb][kb] = s1[qb][kb];
                s1[qb][kb] = ts;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const h8 tp = p0[qb][kb][hh];
                    p0[qb][kb][hh] = p1[qb][kb][hh];
                    p1[qb][kb][hh] = tp;
                }
            }
    }
    for (; t < ntiles; t += 2) {
        general(t, s0, p0, s1, p1);
        if (t + 1 < ntiles) general(t + 1, s1, p1, s0, p0);
    }
    }   // pipelined loop

    // Outputs leave the MFMA accumulators with each lane holding one query
    // and runs of 4 consecutive columns, so direct stores would touch 32 rows
    // per instruction in 8- or 16-byte pieces.  Each wave transposes its block
    // through a private, XOR-swizzled slice of the tile stages instead (idle
    // now: every wave is past its last tile read and no transfer is in
    // flight), then stores whole rows with 16-byte lanes.
    static_assert(sizeof(sKV) >= NW * QB * (SPLIT ? 8192 : 4096), "output staging fits in the tile stages");
    char *const stage_base = reinterpret_cast<char *>(&sKV[0][0][0]);
    if (SPLIT) {
        // Partial result of this slice: the O^T accumulator, the reference
        // max and the row sum (all relative to 2^msc), for the combine step.
        // Rows of 64 fp32 (256 bytes, 16 chunks): lane (c, g2) holds logical
        // chunks 8*db + 2*i + g2 of row c, stored at chunk ^ (c & 15).
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            char *blk = stage_base + 8192 * (QB * wave + qb);
            const float lt = l[qb] + xor32(l[qb]);
            const int q = qw0 + 32 * qb + c;
            const int64_t row0 = ((int64_t)ks * BH + bh) * S + qw0 + 32 * qb;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    f4 x;
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[j] = o[qb][db][4 * i + j];
                    *reinterpret_cast<f4 *>(blk + c * 256 + (((8 * db + 2 * i + g2) ^ (c & 15)) << 4)) = x;
                }
            if (q < S && g2 == 0) *reinterpret_cast<f2 *>(a.part_ml + 2 * (row0 + c)) = f2{msc[qb], lt};
            const int ch = lane & 15;   // lane: chunk ch of rows 4k + (lane >> 4)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int r = 4 * k + (lane >> 4);
                const f4 v = *reinterpret_cast<const f4 *>(blk + r * 256 + ((ch ^ (r & 15)) << 4));
                if (qw0 + 32 * qb + r < S) *reinterpret_cast<f4 *>(a.part_o + (row0 + r) * HD + 4 * ch) = v;
            }
        }
        return;
    }
    // Epilogue: O = acc / l (l == 0 -> 0), LSE = (m*scale2 + log2 l) * ln 2.
    // O rows leave through this wave's 4 KB slice of the stages.
    const bool o16 = ((a.osb | a.osh | a.oss) & 7) == 0;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float lt = l[qb] + xor32(l[qb]);
        const int q = qw0 + 32 * qb + c;
        if (q < S && g2 == 0) Lp[q] = (msc[qb] == -INFINITY) ? -INFINITY : (msc[qb] + log2f(lt)) * LN2;
        // With dropout, P was zeroed but not scaled: 1/(1-p) joins 1/l here.
        const float oscale = lt > 0.f ? (DROPOUT ? a.inv_keep / lt : 1.f / lt) : 0.f;
        store_rows_f16(o[qb][0], o[qb][1], oscale, stage_base + 4096 * (QB * wave + qb),
                       Op + (int64_t)(qw0 + 32 * qb) * a.oss, a.oss, S - (qw0 + 32 * qb), o16);
    }
}

// Merges the slices of a split forward: with M the largest reference max of
// a query's slices and w_s = 2^(m_s - M), O = sum_s w_s O_s / sum_s w_s l_s
// and LSE = (M + log2 sum_s w_s l_s) ln 2 (a query no slice saw: O = 0,
// LSE = -inf).  16 threads per query, 4 of its 64 columns each.
__global__ __launch_bounds__(256) void fwd_combine_kernel(const FwdArgs a) {
    const int S = a.S;
    const int64_t BHS = (int64_t)a.B * a.H * S;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);   // (b*H + h)*S + q
    if (row >= BHS) return;
    const int part = threadIdx.x & 15;
    const int bh = (int)(row / S), q = (int)(row - (int64_t)bh * S);
    const int b = bh / a.H, h = bh - b * a.H;
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.part_ml[2 * (s * BHS + row)]);
    float lsum = 0.f;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
        for (int s = 0; s < a.nsplit; ++s) {
            const f2 ml = *reinterpret_cast<const f2 *>(a.part_ml + 2 * (s * BHS + row));
            if (ml[0] == -INFINITY) continue;
            const float w = __builtin_amdgcn_exp2f(ml[0] - M);
            lsum += w * ml[1];
            const f4 x = *reinterpret_cast<const f4 *>(a.part_o + (s * BHS + row) * HD + 4 * part);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] += w * x[j];
        }
    }
    // inv_keep: 1/(1-p), which the slices left out of their O (1 without dropout).
    const float inv = lsum > 0.f ? a.inv_keep / lsum : 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] *= inv;
    *reinterpret_cast<h4 *>(a.o + b * a.osb + h * a.osh + (int64_t)q * a.oss + 4 * part) =
        __builtin_convertvector(acc, h4);
    if (part == 0)
        a.lse[b * a.lsb + h * a.lsh + q] = (M == -INFINITY || !(lsum > 0.f)) ? -INFINITY : (M + log2f(lsum)) * LN2;
}

// ---------------------------------------------------------------------------
// Decode: one query against Sk keys.  VALU only -- the work is streaming K and
// V from HBM once; an MFMA tile would use one of its 32 query rows.
// ---------------------------------------------------------------------------
// Workgroup (slice ks, b*H + h) takes the keys of slice ks (all keys when
// nsplit = 1), cut into four runs of whole 64-key blocks, one per wave.  Per
// block, lane L = 8g + c8 loads the 16-byte chunk c8 (dims 8*c8 .. +7) of key
// rows k0 + 8i + g, i = 0..7, of K and of V (each of the eight loads covers 1 KB
// of consecutive rows), forms the partial dot of its chunk with q's, and a
// butterfly over the 8 lanes of group g gives all of them the score of row
// 8i + g.  Each lane runs the online softmax over its rows {8i + g} and
// accumulates P V for its 8 dims.  The groups' states merge by shuffles (lanes
// xor 8, 16, 32), the waves' in LDS; the result is O and LSE (nsplit = 1) or
// the slice's partial for fwd_combine_kernel.
constexpr int DEC_NW = 4;

// Sum over the 8 lanes of each aligned group of 8, returned to all of them:
// DPP quad_perm [1,0,3,2] and [2,3,0,1] (partners xor 1, xor 2), then
// row_half_mirror (lane i <-> 7 - i of each 8, which lies in the other quad).
__device__ __forceinline__ float sum8(float x) {
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
    return x;
}

__device__ __forceinline__ void merge_state(float &m, float &l, f8 &acc, float mo, float lo, const f8 &ao) {
    const float mx = fmaxf(m, mo);
    const float wa = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mx);
    const float wb = (mo == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mo - mx);
    l = l * wa + lo * wb;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = acc[e] * wa + ao[e] * wb;
    m = mx;
}

template <bool CAUSAL>
__global__ __launch_bounds__(DEC_NW * 64) void decode_kernel(const FwdArgs a) {
    __shared__ float sm[DEC_NW][HD + 2];   // per wave: O accumulator, max, sum
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 3, c8 = lane & 7;
    const int BH = a.B * a.H;
    const int ks = blockIdx.x / BH, bh = blockIdx.x - ks * BH;
    const int b = bh / a.H, h = bh - b * a.H;
    const int Sk = a.Sk;
    const int kend = CAUSAL ? min(Sk, a.coff + 1) : Sk;   // query 0 sees keys j <= coff
    const int kb = ks * a.split_keys, ke = min(kend, kb + a.split_keys);
    const int nblk = ke > kb ? (ke - kb + 63) / 64 : 0;
    const int per = (nblk + DEC_NW - 1) / DEC_NW;
    const int wb = kb + 64 * min(nblk, wave * per);
    const int we = min(ke, kb + 64 * min(nblk, (wave + 1) * per));
    const _Float16 *Kp = a.k + b * a.ksb + h * a.ksh + 8 * c8;
    const _Float16 *Vp = a.v + b * a.vsb + h * a.vsh + 8 * c8;
    const h8 qv = *reinterpret_cast<const h8 *>(a.q + b * a.qsb + h * a.qsh + 8 * c8);
    const h8 qn = neg_h8_if(qv, a.negate);
    const float scale2 = a.scale2;

    float m = -INFINITY, l = 0.f;
    f8 acc;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    // Block k0's rows are loaded while block k0 - 64 is computed (two register sets).
    h8 kn[8], vn[8];
    auto load = [&](int k0) FA2_INLINE {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = min(k0 + 8 * i + g, Sk - 1);   // rows past the run: loaded in bounds, masked
            kn[i] = *reinterpret_cast<const h8 *>(Kp + (int64_t)r * a.kss);
            vn[i] = *reinterpret_cast<const h8 *>(Vp + (int64_t)r * a.vss);
        }
    };
    if (wb < we) load(wb);
    for (int k0 = wb; k0 < we; k0 += 64) {
        h8 kx[8], vx[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            kx[i] = kn[i];
            vx[i] = vn[i];
        }
        if (k0 + 64 < we) load(k0 + 64);
        float s[8];
        float mx = m;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const h2 qq = {qn[2 * e], qn[2 * e + 1]}, kk = {kx[i][2 * e], kx[i][2 * e + 1]};
                d = __builtin_amdgcn_fdot2(qq, kk, d, false);
            }
            d = sum8(d);
            s[i] = (k0 + 8 * i + g < we) ? d * scale2 : -INFINITY;
            mx = fmaxf(mx, s[i]);
        }
        const float alpha = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mx);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p = (s[i] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(s[i] - mx);
            l += p;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] += p * (float)vx[i][e];
        }
        m = mx;
    }
    // Merge the 8 row groups (lanes with the same c8), then the waves.
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
        f8 ao;
#pragma unroll
        for (int e = 0; e < 8; ++e) ao[e] = __shfl_xor(acc[e], off);
        merge_state(m, l, acc, __shfl_xor(m, off), __shfl_xor(l, off), ao);
    }
    if (g == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sm[wave][8 * c8 + e] = acc[e];
        if (c8 == 0) {
            sm[wave][HD] = m;
            sm[wave][HD + 1] = l;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_NW; ++w) M = fmaxf(M, sm[w][HD]);
    float L = 0.f, o = 0.f;   // lane = dim
    if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < DEC_NW; ++w) {
            const float mw = sm[w][HD];
            if (mw == -INFINITY) continue;
            const float wt = __builtin_amdgcn_exp2f(mw - M);
            L += wt * sm[w][HD + 1];
            o += wt * sm[w][lane];
        }
    }
    if (a.part_o) {   // slice partial: (ks * BH + bh) * S + q with S = 1, q = 0
        const int64_t row = (int64_t)ks * BH + bh;
        a.part_o[row * HD + lane] = o;
        if (lane == 0) *reinterpret_cast<f2 *>(a.part_ml + 2 * row) = f2{M, L};
        return;
    }
    a.o[b * a.osb + h * a.osh + lane] = (_Float16)(L > 0.f ? o / L : 0.f);
    if (lane == 0) a.lse[b * a.lsb + h * a.lsh] = (M == -INFINITY || !(L > 0.f)) ? -INFINITY : (M + log2f(L)) * LN2;
}

#ifndef FA2_FWD_NARROW
#define FA2_FWD_NARROW 1
#endif

template <bool CAUSAL, bool DROPOUT, bool DMASK>
void launch_narrow(const FwdArgs &a, hipStream_t st) {
    const int nqblk = (a.S + qwg_of(1) - 1) / qwg_of(1);
    hipLaunchKernelGGL((fwd_kernel<CAUSAL, DROPOUT, false, DMASK, 1, true>), dim3((unsigned)(nqblk * a.B * a.H)),
                       dim3(NW * 64), 0, st, a);
}

// Workgroup order of the narrow forward (query_block_order): groups of 16
// heads per XCD for sequences of at most 8 narrow query blocks, where a
// head's K / V tiles would otherwise leave the L2 between its query blocks
// (measured at B*S = 32k, H = 12: S = 512 9% faster, S = 1024 5%; S = 2048
// 2% slower, S = 4096 equal); the plain order otherwise.
#ifndef FA2_FWD_GROUP_MAX_S
#define FA2_FWD_GROUP_MAX_S 1024
#endif

template <bool SPLIT>
void launch_fwd_t(const FwdArgs &a_in, bool causal, bool dropout, hipStream_t st) {
    FwdArgs a = a_in;
    a.hgroup = 0;
    const dim3 block(NW * 64);
    // Keep-bit words only from the unsplit forward (the training path).
    const bool dmask = !SPLIT && dropout && a.drop_mask != nullptr;
    // The narrow kernel (one query block per wave, four workgroups per CU)
    // when its grid fills at least one round of those slots: the training
    // shapes (measured at B*S = 32k: 7% faster at S = 4096, 20% at S = 512)
    // and large prefill chunks.  Smaller grids -- prefill chunks of a few
    // hundred queries over long caches, where every workgroup runs the whole
    // key range -- keep the software-pipelined kernel below (the narrow one
    // was 5-16% slower there).
    const int64_t narrow_wgs = (int64_t)((a.S + qwg_of(1) - 1) / qwg_of(1)) * a.B * a.H;
    if (!SPLIT && FA2_FWD_NARROW && narrow_wgs >= (int64_t)NARROW_WAVES * device_cus()) {
        if ((a.B * a.H) % 8 == 0 && a.S <= FA2_FWD_GROUP_MAX_S) a.hgroup = 16;
        if (causal) {
            if (dmask) launch_narrow<true, true, true>(a, st);
            else if (dropout) launch_narrow<true, true, false>(a, st);
            else launch_narrow<true, false, false>(a, st);
        } else {
            if (dmask) launch_narrow<false, true, true>(a, st);
            else if (dropout) launch_narrow<false, true, false>(a, st);
            else launch_narrow<false, false, false>(a, st);
        }
        return;
    }
    // Without key slices or keep-bit words: two query blocks per wave (2 to 3%
    // faster than the pipelined single block) when that still fills every
    // slot of two workgroups per CU; otherwise (short query ranges: prefill
    // chunks) one block per wave, for twice the workgroups.  With keep-bit
    // words the two-block kernel would spill (two words per lane and tile
    // under construction), so they keep one block per wave.
    const bool two = !SPLIT && !dmask &&
                     (int64_t)((a.S + qwg_of(2) - 1) / qwg_of(2)) * a.B * a.H >= 2 * (int64_t)device_cus();
    const int nqblk = (a.S + (two ? qwg_of(2) : qwg_of(1)) - 1) / (two ? qwg_of(2) : qwg_of(1));
    const dim3 grid((unsigned)(nqblk * a.B * a.H * (SPLIT ? a.nsplit : 1)));
    if (causal) {
        if (two) {
            if (dropout)
                hipLaunchKernelGGL((fwd_kernel<true, true, false, false, 2>), grid, block, 0, st, a);
            else
                hipLaunchKernelGGL((fwd_kernel<true, false, false, false, 2>), grid, block, 0, st, a);
        } else if (dmask)
            hipLaunchKernelGGL((fwd_kernel<true, true, SPLIT, !SPLIT, 1>), grid, block, 0, st, a);
        else if (dropout)
            hipLaunchKernelGGL((fwd_kernel<true, true, SPLIT, false, 1>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((fwd_kernel<true, false, SPLIT, false, 1>), grid, block, 0, st, a);
    } else {
        if (two) {
            if (dropout)
                hipLaunchKernelGGL((fwd_kernel<false, true, false, false, 2>), grid, block, 0, st, a);
            else
                hipLaunchKernelGGL((fwd_kernel<false, false, false, false, 2>), grid, block, 0, st, a);
        } else if (dmask)
            hipLaunchKernelGGL((fwd_kernel<false, true, SPLIT, !SPLIT, 1>), grid, block, 0, st, a);
        else if (dropout)
            hipLaunchKernelGGL((fwd_kernel<false, true, SPLIT, false, 1>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((fwd_kernel<false, false, SPLIT, false, 1>), grid, block, 0, st, a);
    }
}

}  // namespace

hipError_t launch_fwd(const FwdArgs &a, bool causal, bool dropout, hipStream_t st) {
    launch_fwd_t<false>(a, causal, dropout, st);
    return hipGetLastError();
}

hipError_t launch_fwd_decode(const FwdArgs &a, bool causal, hipStream_t st) {
    const dim3 grid((unsigned)(a.B * a.H * a.nsplit)), block(DEC_NW * 64);
    if (causal)
        hipLaunchKernelGGL(decode_kernel<true>, grid, block, 0, st, a);
    else
        hipLaunchKernelGGL(decode_kernel<false>, grid, block, 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit <= 1) return e;
    hipLaunchKernelGGL(fwd_combine_kernel, dim3((unsigned)((a.B * a.H + 15) / 16)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_fwd_split(const FwdArgs &a, bool causal, bool dropout, hipStream_t st) {
    launch_fwd_t<true>(a, causal, dropout, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t rows = (int64_t)a.B * a.H * a.S;
    hipLaunchKernelGGL(fwd_combine_kernel, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace fa2
