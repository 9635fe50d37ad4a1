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
//
// Epilogue per 16-row block: one min and one compare per query block decide
// whether any value passes its query's threshold; passing values are
// appended to the (wave, query) list in global memory.  Every query has one
// list per workgroup and each list keeps kk_final entries, so a list cut
// publishes its own kk_final-th value as a bound on the query's shared
// threshold.  The merge, re-rank and verification are those of the other
// scans; lists are laid out [nqblk][nsplit][1][4 * 16 * NQB][cap] and end at
// their counts (list_cnt) instead of being cut to kk_final entries.
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

size_t share_lds_bytes(int nks, int nqb, int rt, int cap) {
    const size_t kp = (size_t)32 * nks + 8, tr = (size_t)16 * rt;
    const size_t stage = tr * kp * 2 + tr * 4;
    return 2 * stage + (size_t)4 * 16 * nqb * 8 + (size_t)4 * cap * 8;
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

    // LDS: two stages [TR][KP] bf16 + [TR] row norms, then the lists'
    // counters and thresholds [BN] and the per-wave sort buffers [4][cap]
    int *cnt = (int *)(smem + 2 * S::STAGE_BYTES);
    float *thr = (float *)(cnt + S::BN);
    float *sv = thr + S::BN;
    int *si = (int *)(sv + S::NW * a.cap);
    const int64_t q0 = qblk * S::BN;
    for (int t = tid; t < S::BN; t += S::NT) {
        cnt[t] = 0;
        thr[t] = q0 + t < a.nq ? VS_INF : -VS_INF;
    }
    const int qw = wave * BNW;  // the wave's first query in the block
    int *cnt_w = cnt + qw;
    float *thr_w = thr + qw;
    float *sv_w = sv + wave * a.cap;
    int *si_w = si + wave * a.cap;
    const int64_t list_base = (qblk * a.nsplit + split) * (int64_t)S::BN * a.cap;
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
    auto gload = [&](int64_t t) __attribute__((always_inline)) {
        // the last tile reads at most TR rows past the end, inside the
        // allocation's slack rows; the resource stops there
        const int64_t lim = min((int64_t)INT32_MAX, (a.n - t + TR) * (int64_t)row_bytes);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)((const char *)a.xb + t * row_bytes), 0, (int)lim, kBufRsrcWord3);
#pragma unroll
        for (int j = 0; j < S::LOADS; ++j) ra[j] = buf_load16(rs, tid * 16, j * S::NT * 16);
        if (l2 && tid < TR / 4) rn = *(const f32x4_t *)(a.xn + t + 4 * tid);
    };
    auto lstore = [&](char *stage) __attribute__((always_inline)) {
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
        if (l2 && tid < TR / 4) *(f32x4_t *)((float *)(As + TR * KP) + 4 * tid) = rn;
    };

    gload(r0);
    lstore(smem);
    __syncthreads();

    float thr_r[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = thr_w[qb * 16 + r16];

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

    const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
    int par = 0;
    for (int64_t t0 = r0; t0 < r1; t0 += TR) {
        const int64_t tn = t0 + TR;
        // rows of the tile inside the split (32-bit: scalar compares below)
        const int rows_in = (int)min((int64_t)TR, r1 - t0);
        const bool more = tn < r1;
        if constexpr (!KMIN) gthr_load();
        if (more) gload(tn);
        const uint16_t *As = (const uint16_t *)(smem + par * S::STAGE_BYTES);
        const float *Ns = (const float *)(As + TR * KP);
        const uint16_t *al = As + r16 * KP + 8 * g;

        // the MFMAs of row block rb + 1 are issued before the epilogue of
        // row block rb, so its compares run while they execute
        auto mma = [&](int rb, f32x4_t (&acc)[NQB]) __attribute__((always_inline)) {
            const f32x4_t init = l2 ? *(const f32x4_t *)(Ns + rb * 16 + 4 * g) : zero4;
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) acc[qb] = init;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const bf16x8_t av =
                    __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(al + rb * 16 * KP + ks * 32));
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb)
                    acc[qb] = mfma_bf16(av, __builtin_bit_cast(bf16x8_t, bq[ks][qb]), acc[qb]);
            }
        };
        auto epi = [&](int rb, f32x4_t (&acc)[NQB]) __attribute__((always_inline)) {
            const int64_t rbase = t0 + rb * 16 + 4 * g;  // the lane's first row
            if (rb * 16 + 16 > rows_in) {  // rows past the split end never qualify
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (rb * 16 + 4 * g + i >= rows_in) {
#pragma unroll
                        for (int qb = 0; qb < NQB; ++qb) acc[qb][i] = VS_INF;
                    }
            }

            if constexpr (TOPMODE) {
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
                return;
            }

            // ---- epilogue of the 16-row block ----
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
            float m4[NQB];
            bool pass = false;
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                m4[qb] = fminf(fminf(acc[qb][0], acc[qb][1]), fminf(acc[qb][2], acc[qb][3]));
                pass |= m4[qb] < thr_r[qb];
            }
            if (!__ballot(pass)) return;
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
        if constexpr (MODE == 0) {
            // a list gains at most 16 entries per row block (four lanes of
            // four rows): one holding more than cap - TR is cut to its kk
            // best before the tile (the planner's cap >= kk + TR), so the
            // row blocks' epilogues never check for room (measured on C2:
            // 2.74 -> 2.49 ms against a check per row block)
            bool need = false;
            int cq[NQB];
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) cq[qb] = cnt_w[qb * 16 + r16];
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) need |= cq[qb] > a.cap - TR;
            if (__ballot(need)) {
                lds_wave_sync();
                for (int q = 0; q < BNW; ++q) {
                    if (cnt_w[q] > a.cap - TR)
                        flush_list(cv + (int64_t)(qw + q) * a.cap, ci + (int64_t)(qw + q) * a.cap,
                                   &cnt_w[q], &thr_w[q], &thr_w[q], S::BN, 1,
                                   &a.gthr[q0 + qw + q], sv_w, si_w, a.cap, a.kk, a.kk_final, 0,
                                   lane);
                }
                lds_wave_sync();
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = fminf(thr_r[qb], thr_w[qb * 16 + r16]);
                lds_wave_sync();
            }
        }
        f32x4_t accs[2][NQB];
        mma(0, accs[0]);
#pragma unroll
        for (int rb = 0; rb < RT; ++rb) {
            if (rb + 1 < RT) mma(rb + 1, accs[(rb + 1) & 1]);
            epi(rb, accs[rb & 1]);
        }
        if constexpr (!KMIN) {
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = fminf(thr_r[qb], dec_order(gt[qb]));
        }
        // the other stage was last read before the previous barrier
        if (more) lstore(smem + (par ^ 1) * S::STAGE_BYTES);
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
    if (plan.kk != plan.kk_final || plan.cap < plan.kk + 16 * plan.tm || plan.lw != 1 ||
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
