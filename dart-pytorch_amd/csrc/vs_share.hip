// vs_share.hip -- the row-shared scan of libvs_hip.so: large query batches
// over short bf16 rows (gfx950).
//
// One workgroup of four waves owns a block of 4 x 16*NQB queries and one
// split of the database rows.  Each wave keeps the B fragments of its own
// 16*NQB queries in registers for the whole kernel (NKS K-steps of 32 bf16
// values: rows of ld = 32*NKS elements).  The split's rows are walked in
// tiles of 16*RT rows; every tile is read from L2 once per workgroup (16-byte
// loads into registers while the previous tile is multiplied), written to
// one of two LDS stages, and multiplied by all 64*NQB queries of the block:
// four times the query reuse per row byte of the streaming scan, whose waves
// each read their own rows.  One barrier per tile.
//
// Operand layout of v_mfma_f32_16x16x32_bf16, as in the streaming scan
// (lane l, r = l % 16, g = l / 16): A lane holds row r, K elements
// 8g..8g+7 of the 32-wide K-step; B lane holds query r, the same K
// elements; D lane holds rows 4g..4g+3 of query r.  The accumulator starts at
// the row norm xn (L2) or 0 (IP) and the queries are bf16 planes of s*q
// (s = -2 for L2, -1 for IP), so it is "smaller is better" for both metrics.
// Rows past the split end start at +inf and never qualify.
//
// Epilogue per 16-row block: one min and one compare per query block decide
// whether any value passes its query's threshold.  The test of row block rb
// runs between the MFMAs of row block rb + 1 (measured on gfx950: VALU work
// placed between independent MFMAs of the same wave costs nearly nothing,
// the same work after them about four cycles an instruction), and the A
// fragments of row block rb + 2 are read from LDS meanwhile.  Passing values
// are appended to lists in global memory.  Top-k lists belong to one lane
// each (lane (r, g) keeps the rows 4g..4g+3 of every block of query r): four
// lists per query and workgroup, counted in registers, appended without
// atomics or branches per value (a store past the end of the lists' buffer
// resource is dropped).  Each keeps kk entries (kk_final, or kk_final / 4
// with the merge's check that no cut list dropped a winner); a list cut
// publishes its kk-th value (kk = kk_final) or the largest of the query's
// four (kk < kk_final) as a bound on the query's shared threshold.  The
// merge, re-rank and verification are those of the other scans; lists are
// laid out [nqblk][nsplit][LW][4 * 16 * NQB][cap] and end at their counts
// (list_cnt) instead of being cut to kk entries.
#include "vs_device.h"

namespace vs {

// ST 1: bf16 rows.  ST 2: fp32 rows whose bf16 rounding (the hi plane) is
// multiplied: the one-pass selection, whose callers widen their margins and
// decide exactly.
template <int ST, int NKS, int NQB, int RT>
struct ShareShape {
    static constexpr int NW = 4, NT = 256;
    static constexpr int LD = 32 * NKS;         // elements per stored row
    static constexpr int ESZ = ST == 1 ? 2 : 4; // bytes per stored element
    static constexpr int KP = LD + 8;           // LDS row stride (bf16 elements)
    static constexpr int TR = 16 * RT;          // rows per tile
    static constexpr int BNW = 16 * NQB;        // queries per wave
    static constexpr int BN = NW * BNW;         // queries per block
    static constexpr int CPR = LD * ESZ / 16;   // 16-byte global chunks per row
    static constexpr int LOADS = TR * CPR / NT; // 16-byte loads per thread and tile
    static constexpr size_t STAGE_BYTES = (size_t)TR * KP * 2 + (size_t)TR * 4;
    static_assert(TR * CPR % NT == 0, "whole loads per thread");
    static_assert(TR / 4 <= NT, "one thread per 4 row norms");
    static_assert(TR <= kRowSlack, "the last tile reads at most kRowSlack rows past the end");
    static_assert(BN <= 256, "query blocks fit the query padding");
};

size_t share_lds_bytes(int nks, int nqb, int rt, int cap, int lw) {
    const size_t kp = (size_t)32 * nks + 8, tr = (size_t)16 * rt;
    const size_t stage = tr * kp * 2 + tr * 4;
    const size_t bn = (size_t)4 * 16 * nqb;
    return 2 * stage + (lw == 1 ? bn * 8 : lw * bn * 4 + 16) + (size_t)4 * cap * 8;
}

// MODE 0: candidate lists as described above.  MODE 2 (threshold estimates
// from a sample of the rows): no lists are kept during the scan; each lane
// keeps the TOPM smallest values it met per query block, sorted in
// registers, and writes them out at the end (4 * TOPM values per query and
// workgroup, ids 0).  The r-th smallest value of their union is the query's
// r-th smallest over the rows whenever no lane met more than TOPM of those r,
// and larger otherwise, never smaller.  MODE 4 (k-means lists): each lane
// appends what lies below its own running minimum + kmin_margin; with
// kmin_init the minimum starts at the query's entry there, a value at or
// above the accumulator of some row of the scan (so at or above the
// smallest accumulator, which is then still appended: every list keeps what
// lies below the smallest accumulator + kmin_margin).
constexpr int kShareTopMEst = 4; // MODE 2: the estimate needs the 16 smallest of a sample
                                 // spread over many lanes; four slots keep insertions cheap

// A buffer store at this byte offset lies past the end of every list
// resource (the block's lists: 4 x 256 x cap x 4 bytes, cap <= 2^12) and is
// dropped.
constexpr int kDropOffset = 0x7FFFFFF0;

template <int ST, int NKS, int NQB, int RT, int MODE>
__global__ __launch_bounds__(256) void share_scan_kernel(ScanKArgs a) {
    using S = ShareShape<ST, NKS, NQB, RT>;
    constexpr int TOPM = kShareTopMEst;
    constexpr int TR = S::TR, KP = S::KP, BNW = S::BNW;
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r16 = lane & 15, g = lane >> 4;

    int64_t split, qblk;
    if (!map_block(a.nqblk, a.nsplit, &split, &qblk)) return;
    const int64_t r0 = split * a.rows_per_split;
    const int64_t r1 = min(a.n, r0 + a.rows_per_split);
    if (r0 >= r1) return;

    // MODE 0: every lane keeps its own list of each of its queries (lane
    // (r16, g) sees rows 4g .. 4g + 3 of every 16-row block): LW = 4 lists
    // per query and workgroup, list (g, q) at [g][q] of the block's lists,
    // its count in a register of its lane (no shared counters, no atomics)
    constexpr bool LANE = MODE == 0;
    constexpr int LW = LANE ? 4 : 1;
    // LDS: two stages [TR][KP] bf16 + [TR] row norms, then the lists'
    // counters [BN] (MODE 0: none) and thresholds [LW][BN], the per-wave
    // sort buffers [4][cap] and (MODE 0) the count of a list being cut [4]
    int *cnt = (int *)(smem + 2 * S::STAGE_BYTES);
    float *thr = (float *)(cnt + (LANE ? 0 : S::BN));
    float *sv = thr + LW * S::BN;
    int *si = (int *)(sv + S::NW * a.cap);
    const int64_t q0 = qblk * S::BN;
    for (int t = tid; t < LW * S::BN; t += S::NT) {
        if (!LANE) cnt[t] = 0;
        thr[t] = q0 + t % S::BN < a.nq ? VS_INF : -VS_INF;
    }
    const int qw = wave * BNW;  // the wave's first query in the block
    int *cnt_w = cnt + qw;
    float *thr_w = thr + qw;
    float *sv_w = sv + wave * a.cap;
    int *si_w = si + wave * a.cap;
    const int64_t list_base = (qblk * a.nsplit + split) * (int64_t)(LW * S::BN) * a.cap;
    float *cv = a.cand_v + list_base;
    int32_t *ci = a.cand_i + list_base;
    const bool l2 = a.metric == 0;

    // MODE 4 with qorder: slot s of the block stands for point qorder[s]
    // (slots past nq for themselves), whose planes, starting minimum, list
    // and count it uses; list of point p: block p / BN, position p % BN.
    // The block's points are kept in LDS for the appends, in the per-wave
    // sort buffers, which k-means lists never use.
    constexpr bool KMIN = MODE == 4;
    int32_t *pidx = (int32_t *)sv;  // [BN] (MODE 4)
    auto point_of = [&](int64_t s) __attribute__((always_inline)) -> int64_t {
        return KMIN && a.qorder && s < a.nq ? (int64_t)a.qorder[s] : s;
    };
    if constexpr (KMIN) {
        if (a.dev_bound) a.kmin_margin = 2.5f * *a.dev_bound;
        static_assert(S::BN <= S::NW * 256, "the points fit the sort buffers (cap >= 256)");
        for (int t = tid; t < S::BN; t += S::NT) pidx[t] = (int32_t)point_of(q0 + t);
    }
    auto list_of = [&](int64_t p) __attribute__((always_inline)) {
        return ((p / S::BN) * a.nsplit + split) * (int64_t)S::BN + p % S::BN;
    };

    // the wave's queries, plane 0, for the whole kernel
    u32x4_t bq[NKS][NQB];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const int64_t qrow = point_of(q0 + qw + qb * 16 + r16);
            bq[ks][qb] = *(const u32x4_t *)(a.qp + (qrow * 2) * a.ld + ks * 32 + 8 * g);
        }

    // global -> register staging of one tile of rows (and its row norms):
    // buffer loads from a per-tile resource, the thread's j-th load NT
    // 16-byte chunks after its first (one offset register for all)
    constexpr int row_bytes = S::LD * S::ESZ;
    u32x4_t ra[S::LOADS];
    f32x4_t rn = {0.f, 0.f, 0.f, 0.f};
    auto rows_rs = [&](int64_t t) __attribute__((always_inline)) {
        // the last tile reads at most TR rows past the end, inside the
        // allocation's slack rows; the resource stops there
        const int64_t lim = min((int64_t)INT32_MAX, (a.n - t + TR) * (int64_t)row_bytes);
        return __builtin_amdgcn_make_buffer_rsrc((void *)((const char *)a.xb + t * row_bytes), 0,
                                                 (int)lim, kBufRsrcWord3);
    };
    auto gload_piece = [&](const __amdgpu_buffer_rsrc_t &rs, int j) __attribute__((always_inline)) {
        ra[j] = buf_load16(rs, tid * 16, j * S::NT * 16);
    };
    auto gload_norms = [&](int64_t t) __attribute__((always_inline)) {
        if (l2 && tid < TR / 4) rn = *(const f32x4_t *)(a.xn + t + 4 * tid);
    };
    auto gload = [&](int64_t t) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = rows_rs(t);
#pragma unroll
        for (int j = 0; j < S::LOADS; ++j) gload_piece(rs, j);
        gload_norms(t);
    };
    // (t: the staged tile's first row)
    auto lstore = [&](char *stage, int64_t t) __attribute__((always_inline)) {
        uint16_t *As = (uint16_t *)stage;
#pragma unroll
        for (int j = 0; j < S::LOADS; ++j) {
            const int i = tid + j * S::NT, row = i / S::CPR, c = i % S::CPR;
            if constexpr (ST == 1) {
                *(u32x4_t *)(As + row * KP + c * 8) = ra[j];
            } else {  // 4 fp32 values -> their bf16 rounding
                typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
                const bf16x4_t hi = __builtin_convertvector(__builtin_bit_cast(f32x4_t, ra[j]), bf16x4_t);
                *(u32x2_t *)(As + row * KP + c * 4) = __builtin_bit_cast(u32x2_t, hi);
            }
        }
        // the accumulators' starting values: the row norms (L2) or 0 (IP),
        // +inf for rows past the split end, which then never qualify (set
        // here, where the loads have been waited for anyway)
        if (tid < TR / 4) {
            f32x4_t v = l2 ? rn : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (t + 4 * tid + i >= r1) v[i] = VS_INF;
            *(f32x4_t *)((float *)(As + TR * KP) + 4 * tid) = v;
        }
    };

    gload(r0);
    lstore(smem, r0);
    __syncthreads();

    float thr_r[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = thr_w[(LANE ? g * S::BN : 0) + qb * 16 + r16];
    // MODE 0: the lane's list counts, and its lists' stores: buffer stores
    // at 32-bit offsets from the block's lists (element lofs + qb 16 cap +
    // count of list (g, qw + 16 qb + r16))
    int lcnt[LANE ? NQB : 1];
#pragma unroll
    for (int qb = 0; qb < (LANE ? NQB : 1); ++qb) lcnt[qb] = 0;
    const int lofs = (g * S::BN + qw + r16) * a.cap;
    const int lbytes = LW * S::BN * a.cap * 4;
    const __amdgpu_buffer_rsrc_t rs_v =
        __builtin_amdgcn_make_buffer_rsrc((void *)cv, 0, lbytes, kBufRsrcWord3);
    const __amdgpu_buffer_rsrc_t rs_i =
        __builtin_amdgcn_make_buffer_rsrc((void *)ci, 0, lbytes, kBufRsrcWord3);

    // the shared thresholds are read at the start of a tile and applied at
    // its end, when the read has long completed
    uint32_t gt[NQB];
    auto gthr_load = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb)
            gt[qb] = __hip_atomic_load(&a.gthr[q0 + qw + qb * 16 + r16], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    };
    // MODE 4 (k-means lists) keeps its thresholds to itself: each lane
    // appends what lies below its own running minimum + kmin_margin
    float best_r[KMIN ? NQB : 1];
#pragma unroll
    for (int qb = 0; qb < (KMIN ? NQB : 1); ++qb)
        best_r[qb] = KMIN && a.kmin_init ? a.kmin_init[point_of(q0 + qw + qb * 16 + r16)] : VS_INF;
    if constexpr (!KMIN) {
        gthr_load();
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = fminf(thr_r[qb], dec_order(gt[qb]));
    }

    constexpr bool TOPMODE = MODE == 2;
    float top[TOPMODE ? NQB : 1][TOPM];
#pragma unroll
    for (int qb = 0; qb < (TOPMODE ? NQB : 1); ++qb)
#pragma unroll
        for (int m = 0; m < TOPM; ++m) top[qb][m] = VS_INF;

    int par = 0;
    for (int64_t t0 = r0; t0 < r1; t0 += TR) {
        const int64_t tn = t0 + TR;
        const bool more = tn < r1;
        if constexpr (!KMIN) gthr_load();
        // the next tile's loads: all at once for short tiles, else spread
        // over the first half of the row blocks (two per row block), so the
        // tile's first MFMAs do not wait behind a burst of loads (C2 scan
        // 2.25 -> 2.22 ms); they are written to LDS at the tile's end
        constexpr bool SPL = RT >= 4;
        const __amdgpu_buffer_rsrc_t rs_n = rows_rs(tn);
        if (!SPL && more) gload(tn);
        if (SPL && more) gload_norms(tn);
        const uint16_t *As = (const uint16_t *)(smem + par * S::STAGE_BYTES);
        const float *Ns = (const float *)(As + TR * KP);
        const uint16_t *al = As + r16 * KP + 8 * g;

        // a row block's A fragments and starting values, read from LDS one
        // row block ahead of its MFMAs where the registers allow that at two
        // waves per SIMD (up to 16 MFMAs per row block), else just before
        // them (and the order of the MFMAs and the pass test is left to the
        // compiler)
        constexpr bool PREF = NKS * NQB <= 16;
        auto frag = [&](int rb, u32x4_t (&af)[NKS], f32x4_t &init) __attribute__((always_inline)) {
            init = *(const f32x4_t *)(Ns + rb * 16 + 4 * g);
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) af[ks] = *(const u32x4_t *)(al + rb * 16 * KP + ks * 32);
        };
        auto mma = [&](const u32x4_t (&af)[NKS], const f32x4_t &init, f32x4_t (&acc)[NQB])
                       __attribute__((always_inline)) {
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) acc[qb] = init;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
                    acc[qb] = mfma_bf16(__builtin_bit_cast(bf16x8_t, af[ks]),
                                        __builtin_bit_cast(bf16x8_t, bq[ks][qb]), acc[qb]);
        };
        auto topm = [&](f32x4_t (&acc)[NQB]) __attribute__((always_inline)) {
            // the four smallest of the lane's four (sorted) and its four
            // new values, branch-free: sort the new ones (five
            // compare-exchanges), pair the two sorted runs head to tail
            // (the smaller of each pair: a bitonic run holding the four
            // smallest), sort that (four compare-exchanges).  While the
            // slots fill, nearly every wave has a lane taking each value,
            // where a per-value insertion cost four compare-exchanges.
            static_assert(TOPM == 4, "a merge of two sorted runs of four");
            auto cx = [](float &x, float &y) __attribute__((always_inline)) {
                const float lo = fminf(x, y);
                y = fmaxf(x, y);
                x = lo;
            };
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                float v0 = acc[qb][0], v1 = acc[qb][1], v2 = acc[qb][2], v3 = acc[qb][3];
                if (!__ballot(fminf(fminf(v0, v1), fminf(v2, v3)) < top[qb][3])) continue;
                cx(v0, v1);
                cx(v2, v3);
                cx(v0, v2);
                cx(v1, v3);
                cx(v1, v2);
                float c0 = fminf(top[qb][0], v3), c1 = fminf(top[qb][1], v2);
                float c2 = fminf(top[qb][2], v1), c3 = fminf(top[qb][3], v0);
                cx(c0, c2);
                cx(c1, c3);
                cx(c0, c1);
                cx(c2, c3);
                top[qb][0] = c0;
                top[qb][1] = c1;
                top[qb][2] = c2;
                top[qb][3] = c3;
            }
        };

        // the pass test of a row block: branch-free, its VALU instructions
        // scheduled between the next row block's MFMAs
        auto check = [&](f32x4_t (&acc)[NQB], float (&m4)[NQB]) __attribute__((always_inline)) {
            if constexpr (KMIN) {
                // the lane's own running minimum (rows 4g .. 4g + 3 of every
                // block): an accumulator of a scanned row, so at or above the
                // query's smallest, which is all the lists need (the minimum
                // over the query's four lanes is tighter by little and costs
                // two cross-row swaps per block: 5 % of the scan on C4)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    const float m =
                        fminf(fminf(acc[qb][0], acc[qb][1]), fminf(acc[qb][2], acc[qb][3]));
                    best_r[qb] = fminf(best_r[qb], m);
                    thr_r[qb] = fminf(thr_r[qb], best_r[qb] + a.kmin_margin);
                }
            }
            bool pass = false;
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                m4[qb] = fminf(fminf(acc[qb][0], acc[qb][1]), fminf(acc[qb][2], acc[qb][3]));
                pass |= m4[qb] < thr_r[qb];
            }
            return pass;
        };
        // one query block's share of the pass test (the same as check's)
        auto check_qb = [&](f32x4_t (&acc)[NQB], float (&m4)[NQB], int qb)
                            __attribute__((always_inline)) -> bool {
            const float m = fminf(fminf(acc[qb][0], acc[qb][1]), fminf(acc[qb][2], acc[qb][3]));
            if constexpr (KMIN) {
                best_r[qb] = fminf(best_r[qb], m);
                thr_r[qb] = fminf(thr_r[qb], best_r[qb] + a.kmin_margin);
            }
            m4[qb] = m;
            return m < thr_r[qb];
        };
        // row block rb + 1's MFMAs with row block rb's pass test and row
        // block rb + 2's fragment reads between them, in a pinned order: the
        // test's VALU instructions and the reads issue while the MFMAs run
        auto mma_check = [&](const u32x4_t (&af)[NKS], const f32x4_t &init, f32x4_t (&acc)[NQB],
                             f32x4_t (&prev)[NQB], float (&m4)[NQB], int rbf,
                             u32x4_t (&afn)[NKS], f32x4_t &initn) __attribute__((always_inline)) {
            bool pass = false;
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) acc[qb] = init;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    const int j = ks * NQB + qb;
                    acc[qb] = mfma_bf16(__builtin_bit_cast(bf16x8_t, af[ks]),
                                        __builtin_bit_cast(bf16x8_t, bq[ks][qb]), acc[qb]);
                    if (rbf >= 0) {
                        if (j == 0) initn = *(const f32x4_t *)(Ns + rbf * 16 + 4 * g);
                        else if (j <= NKS)
                            afn[j - 1] = *(const u32x4_t *)(al + rbf * 16 * KP + (j - 1) * 32);
                    }
                    if (j % NKS == 0) pass |= check_qb(prev, m4, j / NKS);
                    if constexpr (PREF) __builtin_amdgcn_sched_barrier(0);
                }
            return pass;
        };
        // the appends of a row block with passing values
        auto epi = [&](int rb, f32x4_t (&acc)[NQB], const float (&m4)[NQB])
                       __attribute__((always_inline)) {
            const int64_t rbase = t0 + rb * 16 + 4 * g;  // the lane's first row
            // k-means lists: one that may gain entries here (at most 16: four
            // lanes of four rows) and holds more than cap - 16 is marked
            // full, count cap + 1 (its point goes to the exhaustive search).
            // The counts live in LDS; only lanes with a passing value read
            // them.  (Top-k lists are cut before each tile instead.)
            if constexpr (KMIN) {
                bool need = false;
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
                    if (m4[qb] < thr_r[qb]) need |= cnt_w[qb * 16 + r16] > a.cap - 16;
                if (__ballot(need)) {
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb) {
                        const int q = qb * 16 + r16;
                        if (cnt_w[q] > a.cap - 16) {
                            thr_r[qb] = -VS_INF;
                            if (g == 0) cnt_w[q] = a.cap + 1;
                        }
                    }
                    lds_wave_sync();
                }
            }
            if constexpr (LANE) {
                // appends to the lane's own lists, at their counts, without
                // branches: every lane stores, and the stores of values that
                // do not pass go past the end of the lists' buffer resource,
                // which drops them
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    if (!__ballot(m4[qb] < thr_r[qb])) continue;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // (copied out of the vector first: a bit cast of a
                        // vector element reads element 0)
                        const float v = acc[qb][i];
                        const bool p = v < thr_r[qb];
                        const int off = p ? (lofs + qb * 16 * a.cap + lcnt[qb]) * 4 : kDropOffset;
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rs_v,
                                                              off, 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(rbase + i), rs_i, off, 0,
                                                              0);
                        lcnt[qb] += p ? 1 : 0;
                    }
                }
                return;
            }
            // appends: each lane with passing values reserves its slots with
            // one LDS atomic on its query's count (passing values are rare:
            // most query blocks of a row block have none)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                if (!__ballot(m4[qb] < thr_r[qb])) continue;
                int c = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) c += acc[qb][i] < thr_r[qb] ? 1 : 0;
                if (c > 0) {
                    const int q = qw + qb * 16 + r16;
                    int pos = atomicAdd(&cnt_w[qb * 16 + r16], c);
                    const int64_t lq = KMIN ? list_of(pidx[q]) * a.cap
                                            : list_base + (int64_t)q * a.cap;
                    float *cvq = a.cand_v + lq;
                    int32_t *ciq = a.cand_i + lq;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (acc[qb][i] < thr_r[qb]) {
                            cvq[pos] = acc[qb][i];
                            ciq[pos] = (int32_t)(rbase + i);
                            ++pos;
                        }
                    }
                }
            }
            lds_wave_sync();
        };
        if constexpr (LANE) {
            // a lane's list gains at most 4 entries per row block: one
            // holding more than cap - 4 RT is cut to its kk best before the
            // tile (the planner's cap >= kk + 4 RT), so the row blocks'
            // epilogues never check for room.  The cut (flush_list, one list
            // at a time) reads the counts from LDS.
            bool need = false;
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) need |= lcnt[qb] > a.cap - 4 * RT;
            if (__ballot(need)) {
                int *ccw = si + S::NW * a.cap + wave;
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    for (int l = 0; l < 64; ++l) {  // list (l / 16, qw + 16 qb + l % 16)
                        const int c = __builtin_amdgcn_readlane(lcnt[qb], l);
                        if (c <= a.cap - 4 * RT) continue;
                        const int q = qw + qb * 16 + (l & 15), li = (l >> 4) * S::BN + q;
                        if (lane == 0) *ccw = c;
                        lds_wave_sync();
                        flush_list(cv + (int64_t)li * a.cap, ci + (int64_t)li * a.cap, ccw,
                                   &thr[li], &thr[q], S::BN, LW, &a.gthr[q0 + q], sv_w, si_w,
                                   a.cap, a.kk, a.kk_final, a.publish_block, lane);
                        const int cn = *ccw;
                        if (lane == l) {
                            lcnt[qb] = cn;
                            thr_r[qb] = fminf(thr_r[qb], thr[li]);
                        }
                        lds_wave_sync();
                    }
                }
            }
        }
        f32x4_t accs[2][NQB];
        u32x4_t afr[2][NKS];
        f32x4_t ini[2];
        frag(0, afr[0], ini[0]);
        mma(afr[0], ini[0], accs[0]);
        if constexpr (PREF && RT > 1) frag(1, afr[1], ini[1]);
#pragma unroll
        for (int rb = 0; rb < RT; ++rb) {
            const int c = rb & 1, n = c ^ 1;
            if (SPL && more) {
                constexpr int H = RT / 2;
#pragma unroll
                for (int j = 0; j < S::LOADS; ++j)
                    if (j * H / S::LOADS == rb) gload_piece(rs_n, j);
            }
            if (!PREF && rb + 1 < RT) frag(rb + 1, afr[n], ini[n]);
            if constexpr (TOPMODE) {
                if (rb + 1 < RT) mma(afr[n], ini[n], accs[n]);
                if (PREF && rb + 2 < RT) frag(rb + 2, afr[c], ini[c]);
                topm(accs[c]);
            } else {
                float m4[NQB];
                const bool pass =
                    rb + 1 < RT ? mma_check(afr[n], ini[n], accs[n], accs[c], m4,
                                            PREF && rb + 2 < RT ? rb + 2 : -1, afr[c], ini[c])
                                : check(accs[c], m4);
                if (__ballot(pass)) epi(rb, accs[c], m4);
            }
        }
        if constexpr (!KMIN) {
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = fminf(thr_r[qb], dec_order(gt[qb]));
        }
        // the other stage was last read before the previous barrier
        if (more) lstore(smem + (par ^ 1) * S::STAGE_BYTES, tn);
        __syncthreads();
        par ^= 1;
    }

    if constexpr (TOPMODE) {
        // lane (r16, g) writes its TOPM values of query qw + 16 qb + r16 to
        // slots [g * TOPM, (g + 1) * TOPM) of that query's list (ids 0)
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            const int q = qw + qb * 16 + r16;
            float *cvq = cv + (int64_t)q * a.cap + g * TOPM;
            int32_t *ciq = ci + (int64_t)q * a.cap + g * TOPM;
#pragma unroll
            for (int m = 0; m < TOPM; ++m) {
                cvq[m] = top[qb][m];
                ciq[m] = 0;
            }
        }
        int32_t *lc = a.list_cnt + (qblk * a.nsplit + split) * (int64_t)S::BN + qw;
        for (int q = lane; q < BNW; q += 64) lc[q] = 4 * TOPM;
        if (lane == 0) atomicMax(a.list_cnt + a.nqblk * a.nsplit * S::BN, 4 * TOPM);
        return;
    }
    // final: the lists' entry counts for the merge (which filters by the
    // final shared threshold and keeps the kk_final best itself)
    wave_sync();
    if constexpr (LANE) {
        // counts and own thresholds of the lane's lists, and the largest
        // count (after all lists, for the merge)
        const int64_t lb = (qblk * a.nsplit + split) * (int64_t)(LW * S::BN);
        const int lq = g * S::BN + qw + r16;
        int mx = 0;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            a.list_cnt[lb + lq + qb * 16] = lcnt[qb];
            if (a.lbound) a.lbound[lb + lq + qb * 16] = thr[lq + qb * 16];
            mx = max(mx, lcnt[qb]);
        }
        for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
        if (lane == 0) atomicMax(a.list_cnt + a.nqblk * a.nsplit * (LW * S::BN), mx);
        return;
    }
    if (a.list_cnt) {
        // counts, and the largest one (after all lists, for the merge)
        int32_t *lc = a.list_cnt + (qblk * a.nsplit + split) * (int64_t)S::BN + qw;
        int mx = 0;
        for (int q = lane; q < BNW; q += 64) {
            if (KMIN)
                a.list_cnt[list_of(pidx[qw + q])] = cnt_w[q];
            else
                lc[q] = cnt_w[q];
            mx = max(mx, cnt_w[q]);
        }
        for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
        if (lane == 0) atomicMax(a.list_cnt + a.nqblk * a.nsplit * S::BN, mx);
        return;
    }
    // or: every list holds its kk best in slots [0, kk), padded
    for (int q = 0; q < BNW; ++q) {
        const int c = cnt_w[q];
        float *cvq = cv + (int64_t)(qw + q) * a.cap;
        int32_t *ciq = ci + (int64_t)(qw + q) * a.cap;
        if (c > a.kk) {
            flush_list(cvq, ciq, &cnt_w[q], &thr_w[q], &thr_w[q], S::BN, 1, &a.gthr[q0 + qw + q],
                       sv_w, si_w, a.cap, a.kk, a.kk_final, 0, lane);
        } else {
            for (int j = c + lane; j < a.kk; j += 64) {
                cvq[j] = VS_INF;
                ciq[j] = -1;
            }
        }
    }
}

// mode 4 (the k-means assign) is built for the one-pass selection: fp32
// rows (storage 2), or for 256-element rows their bf16 copy (storage 1)
template <int ST, int NKS, int NQB, int RT>
static void (*share_kmin_kernel())(ScanKArgs) {
    if constexpr (ST == 2 || NKS == 8)
        return share_scan_kernel<ST, NKS, NQB, RT, 4>;
    else
        return nullptr;
}

// The built shapes: X(storage, K-steps, 16-query blocks per wave, 16-row
// blocks per tile).
#define VS_SHARE_SHAPES(X) \
    X(1, 4, 4, 4) X(1, 8, 2, 4) X(2, 4, 4, 2) X(2, 8, 2, 2) X(1, 8, 2, 2) X(1, 4, 4, 8) X(1, 8, 4, 2)

// mode: 0 lists, 2 top-m values, 4 k-means lists
static void (*share_kernel(int st, int nks, int bn, int rt, int64_t ld, int mode))(ScanKArgs) {
#define VS_SHARE_PICK(ST_, NKS_, NQB_, RT_)                                                     \
    if (st == ST_ && nks == NKS_ && bn == 64 * NQB_ && rt == RT_ && ld == 32 * NKS_)              \
        return mode == 4   ? share_kmin_kernel<ST_, NKS_, NQB_, RT_>()                             \
               : mode == 2 ? share_scan_kernel<ST_, NKS_, NQB_, RT_, 2>                           \
                           : share_scan_kernel<ST_, NKS_, NQB_, RT_, 0>;
    VS_SHARE_SHAPES(VS_SHARE_PICK)
#undef VS_SHARE_PICK
    return nullptr;
}

int share_topm_est() { return kShareTopMEst; }

// Workgroups of the shape that one CU holds at once (registers and LDS).
int share_blocks_per_cu(int st, int nks, int bn, int rt, int64_t ld, size_t lds, int mode) {
    void (*fn)(ScanKArgs) = share_kernel(st, nks, bn, rt, ld, mode);
    if (!fn) return 0;
    if (lds > 64 * 1024 && hipFuncSetAttribute((const void *)fn,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds) != hipSuccess)
        return 0;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, 256, lds) != hipSuccess) return 0;
    return nb;
}

hipError_t launch_share_scan(const ScanPlan &plan, const ScanKArgs &args, hipStream_t st) {
    // lists: one per lane (four per query and workgroup) for top-k lists,
    // each gaining up to 4 entries per row block; else one per query (k-means
    // lists, estimates), keeping kk_final
    const bool lane_lists = !plan.share_topm && !plan.share_kmin;
    if (lane_lists ? (plan.lw != 4 || plan.cap < plan.kk + 4 * plan.tm || plan.cap > 4096)
                   : (plan.lw != 1 || plan.kk != plan.kk_final ||
                      plan.cap < plan.kk + 16 * plan.tm) ||
        !args.list_cnt)
        return hipErrorInvalidValue;
    if (plan.share_topm && (plan.share_topm != kShareTopMEst || plan.cap < 4 * plan.share_topm))
        return hipErrorInvalidValue;
    const int64_t total = plan.nqblk * plan.nsplit;
    const int64_t grid = ((total + 7) / 8) * 8;
    if (plan.share_kmin && (plan.share_topm || !(plan.kmin_margin > 0.f || plan.dev_bound)))
        return hipErrorInvalidValue;
    const int mode = plan.share_kmin ? 4 : plan.share_topm ? 2 : 0;
    void (*fn)(ScanKArgs) =
        share_kernel(plan.tile_st, plan.nks, plan.bn, plan.tm, args.ld, mode);
    if (!fn) return hipErrorInvalidValue;
    const size_t lds = plan.lds_bytes;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(256), lds, st, args);
    return hipGetLastError();
}

}  // namespace vs
