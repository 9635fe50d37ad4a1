// vs_gemm.hip -- the GEMM-tiled distance scan of libvs_hip.so for large
// query batches (gfx950).
//
// One workgroup of WR x WQ waves owns a block of BQ = WQ*32*QB queries and
// one split of the database rows, which it walks in row tiles of BR =
// WR*32*RB rows.  Per K-chunk of KC elements both operands are staged in LDS:
// the tile's database rows (A) and the block's prepared query planes (B),
// each loaded once per workgroup with 16-byte global loads, so every byte
// read from L2 feeds BQ queries (rows) or BR rows (queries).  Wave (wr, wq)
// multiplies rows wr*32*RB .. +32*RB by queries wq*32*QB .. +32*QB with
// v_mfma_f32_32x32x16_bf16, holding QB x RB accumulator blocks of 32 x 32.
// Two LDS stages: while the waves multiply one K-chunk, the next chunk's
// global loads are in flight in registers; they are written to the other
// stage after the multiply, and one barrier per chunk orders the two.
//
// Operands follow the convention of the other scans (vs_kernels.hip): the
// queries are bf16 planes of s*q (s = -2 for L2, -1 for IP) and the
// accumulator starts at the row norm xn (L2) or 0 (IP), so it is "smaller is
// better" for both metrics.  fp32 rows are split into bf16 hi and lo planes
// when they are written to LDS; the products are hi*q0 + lo*q0 (+ hi*q1 when
// the queries need a second plane).  Storage code 2 is the one-pass selection
// of fp32 rows: only the bf16 hi plane of the rows and the first query plane
// are multiplied (the callers widen their margins and re-test exactly).  The row norms of a tile travel with its
// first K-chunk.
//
// Epilogue per row tile: per-(row wave, query) candidate lists in global
// memory with per-query shared thresholds (MODE 0), or range appends (MODE
// 1), read by the same merge, re-rank, k-means and range kernels as the
// other scans.  The full distance matrix is never written.
#include <limits.h>

#include <algorithm>

#include <type_traits>

#include "vs_device.h"

namespace vs {

template <int ST, int PB, int WR, int WQ, int RB, int QB, int KC>
struct GemmShape {
    static constexpr int NW = WR * WQ, NT = 64 * NW;
    static constexpr int BR = WR * 32 * RB, BQ = WQ * 32 * QB;
    static constexpr int AP = ST == 0 ? 2 : 1;  // row planes in LDS: bf16 hi (, lo)
    // K-chunk 64: unpadded 128-byte LDS rows whose eight 16-byte pieces are
    // stored XOR-swizzled (piece c of row r at c ^ ((r >> 1) & 7)).  The LDS
    // serves 256 bytes (64 banks) per cycle, so a 16-byte fragment read is
    // conflict-free when 16 consecutive lanes -- rows r .. r + 15, the same
    // logical piece -- hit 16 distinct 16-byte bank groups; a row's group is
    // 8 (r & 1) + physical piece, hence the swizzle by r >> 1 (by r & 7 rows
    // r and r + 8 collide).  Row writes (8 lanes per row) stay conflict-free
    // too.  Smaller chunks pad each row by 16 bytes instead.
    static constexpr bool SW = KC == 64;
    static constexpr int KP = SW ? KC : KC + 8;  // LDS row stride in elements
    static constexpr int ESZ = ST == 1 ? 2 : 4;  // bytes per stored element
    static constexpr int A_CPR = KC * ESZ / 16;  // 16-byte global chunks per row and K-chunk
    static constexpr int A_LOADS = BR * A_CPR / NT;
    static constexpr int B_CPR = KC * 2 / 16;  // 16-byte chunks per query plane and K-chunk
    static constexpr int B_LOADS = BQ * PB * B_CPR / NT;
    static constexpr int STAGE_ELEMS = (AP * BR + PB * BQ) * KP;
    static constexpr size_t STAGE_BYTES = (size_t)STAGE_ELEMS * 2 + (size_t)BR * 4;
    static_assert(KC % 16 == 0, "K-chunk is whole MFMA K-steps");
    static_assert(BR * A_CPR % NT == 0 && BQ * PB * B_CPR % NT == 0, "whole loads per thread");
    static_assert(BR / 4 <= NT, "one thread per 4 row norms");
    static_assert(BR <= kRowSlack, "the last row tile reads at most kRowSlack rows past the end");
    static_assert((KP * 2) % 16 == 0, "16-byte aligned LDS rows");
    static_assert(!SW || KC * 2 / 16 == 8, "the swizzle permutes 8 pieces per row");
};

size_t gemm_lds_bytes(int st, int pb, int wr, int wq, int rb, int qb, int kc, int cap) {
    const size_t br = (size_t)wr * 32 * rb, bq = (size_t)wq * 32 * qb;
    const size_t kp = kc == 64 ? (size_t)kc : (size_t)kc + 8;
    const size_t stage = ((st == 0 ? 2 : 1) * br + (size_t)pb * bq) * kp * 2 + br * 4;
    return 2 * stage + (size_t)wr * bq * 8 + (size_t)wr * wq * cap * 8;  // st 2: one hi plane
}

// Bits v (0..15) of the values of a 32-row block whose row offsets
// 8 (v / 4) + v % 4 + (the lane's 4 h + 32 rb) lie below t, given t minus
// that lane offset: the offsets grow with v, so the bits form a prefix.  The
// epilogues mask their hits with it instead of comparing every offset (per
// value compares are hoisted by the compiler into 64 lane masks per tile).
// Bit v (0..15) set where x[v] < t (LT) or x[v] <= t.  Each compare selects
// an inline constant with the sign bit set or zero, and a funnel shift moves
// that bit in below the bits of the values after it, so no per-bit constant
// is held in a register across the epilogue.
template <bool LT>
__device__ __forceinline__ uint32_t value_mask16(const f32x16_t &x, float t) {
    uint32_t m = 0u;
#pragma unroll
    for (int v = 15; v >= 0; --v) {
        const float xv = x[v];
        const bool p = LT ? xv < t : xv <= t;
        m = __builtin_amdgcn_alignbit(m, p ? 0xbf800000u : 0u, 31);
    }
    return m;
}

__device__ __forceinline__ uint32_t rows_below_mask(int t) {
    int c = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) c += min(max(t - 8 * g, 0), 4);
    return c >= 16 ? 0xffffu : (1u << c) - 1u;
}

// Epilogue of one row tile (shared by both kernels).  Lane (l32, h) of wave
// (wr, wq) holds query qw0 + 32 qb + l32 and, in register v of row block rb,
// row wr0 + 32 rb + 8 (v / 4) + 4 h + v % 4.
struct EpiCtx {
    int64_t q0, r1;
    int qw0, l32, h, lane;
    int *cnt, *cnt_w;
    float *thr, *thr_w, *sv_w;
    int *si_w;
    float *cv;
    int32_t *ci;
};

template <int WR, int BQ, int RB, int QB, int MODE>
__device__ __forceinline__ void gemm_epilogue(f32x16_t (&acc)[QB][RB], const ScanKArgs &a,
                                              const EpiCtx &e, int64_t wr0, float (&thr_r)[QB],
                                              const uint32_t (&gt)[QB], bool &seeded) {
    const int64_t q0 = e.q0, r1 = e.r1;
    const int qw0 = e.qw0, l32 = e.l32, h = e.h, lane = e.lane;
    int *cnt_w = e.cnt_w;
    float *thr = e.thr, *thr_w = e.thr_w, *sv_w = e.sv_w;
    int *si_w = e.si_w;
    float *cv = e.cv;
    int32_t *ci = e.ci;
    (void)gt;
    (void)seeded;
    // ---- epilogue of the tile; lane (l32, h) holds query
    // qw0 + 32 qb + l32 and, in register v of row block rb, row
    // wr0 + 32 rb + 8 (v / 4) + 4 h + v % 4 ----
    // rows past the split end (the last tile only) never qualify:
    // the rare append paths test the row offset against lim; the
    // fast min/ballot test may pass on them, which only costs time
    const int lim = (int)min((int64_t)(32 * RB), r1 - wr0);
    if constexpr (MODE == 0) {
        if (!seeded && lim == 32 * RB) {
            // First tile: instead of appending every value while the
            // lists have no threshold, each lane takes T_lane, the largest
            // of the minima of G groups of its 16 RB values (G = RB, 2 RB,
            // 4 RB, 8 RB or 16 RB, the first >= ceil(kk / 2)): at least
            // ceil(kk / 2) of its values lie at or below T_lane.  The list of
            // (row wave, query) -- two lanes, h = 0 and 1 -- then holds >= kk
            // values at or below T, the larger of the two, once the append
            // below has taken every value < T' (T' the next value code above
            // T); T' becomes the list's threshold.  (The fewest groups that
            // suffice give the tightest threshold.)
            const int need = (a.kk + 1) / 2;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                float tl = -VS_INF;
                if (need <= RB) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        float m = acc[qb][rb][0];
#pragma unroll
                        for (int v = 1; v < 16; ++v) m = fminf(m, acc[qb][rb][v]);
                        tl = fmaxf(tl, m);
                    }
                } else if (need <= 2 * RB) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int u = 0; u < 2; ++u) {
                            float m = acc[qb][rb][8 * u];
#pragma unroll
                            for (int v = 1; v < 8; ++v) m = fminf(m, acc[qb][rb][8 * u + v]);
                            tl = fmaxf(tl, m);
                        }
                } else if (need <= 4 * RB) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            tl = fmaxf(tl, fminf(fminf(acc[qb][rb][4 * u], acc[qb][rb][4 * u + 1]),
                                                 fminf(acc[qb][rb][4 * u + 2], acc[qb][rb][4 * u + 3])));
                } else if (need <= 8 * RB) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int u = 0; u < 8; ++u)
                            tl = fmaxf(tl, fminf(acc[qb][rb][2 * u], acc[qb][rb][2 * u + 1]));
                } else {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int v = 0; v < 16; ++v) tl = fmaxf(tl, acc[qb][rb][v]);
                }
                const float tv = fmaxf(tl, __shfl_xor(tl, 32));
                const int q = qw0 + qb * 32 + l32;
                if (q0 + q < a.nq) {
                    const float t1 = dec_order(enc_order(tv) + 1u);
                    if (h == 0) thr_w[q] = fminf(thr_w[q], t1);
                    thr_r[qb] = fminf(thr_r[qb], t1);
                }
            }
            seeded = true;
        }
        // appends first, then the cuts: every list starts the tile with at
        // most cap - 32 RB entries (a query gains at most 32 * RB per tile
        // from this wave), and a list past that or past its flush point is
        // cut to its kk best after the appends, when no accumulator is live
        // any more (a cut also tightens the list's threshold)
        uint32_t appended = 0u;  // query blocks of this wave that appended
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            thr_r[qb] = fminf(thr_r[qb], dec_order(gt[qb]));
            float m = VS_INF;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int v = 0; v < 16; ++v) m = fminf(m, acc[qb][rb][v]);
            if (!__ballot(m < thr_r[qb])) continue;
            appended |= 1u << qb;
            const int q = qw0 + qb * 32 + l32;
            // the passing values of each 32-row block as a bit mask in a
            // VGPR (no lane mask per value stays live across the append)
            uint32_t mk[RB];
            int c = 0;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                mk[rb] = value_mask16<true>(acc[qb][rb], thr_r[qb]);
                mk[rb] &= rows_below_mask(lim - rb * 32 - 4 * h);
                c += __builtin_popcount(mk[rb]);
            }
            if (c > 0) {
                int pos = atomicAdd(&cnt_w[q], c);
                float *cvq = cv + (int64_t)q * a.cap;
                int32_t *ciq = ci + (int64_t)q * a.cap;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        if ((mk[rb] >> v) & 1u) {
                            cvq[pos] = acc[qb][rb][v];
                            ciq[pos] = (int32_t)(wr0 + rb * 32 + 8 * (v / 4) + 4 * h + v % 4);
                            ++pos;
                        }
                    }
            }
        }
        if (appended) {
            lds_wave_sync();  // the counts' atomics are done
            const int room = min(a.cap - 32 * RB, a.flush_at);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                if (!(appended & (1u << qb))) continue;
                const int q = qw0 + qb * 32 + l32;
                if (!__ballot(h == 0 && cnt_w[q] > room)) continue;
                for (int j = 0; j < 32; ++j) {
                    const int qq = qw0 + qb * 32 + j;
                    if (cnt_w[qq] > room)
                        flush_list(cv + (int64_t)qq * a.cap, ci + (int64_t)qq * a.cap,
                                   &cnt_w[qq], &thr_w[qq], &thr[qq], BQ, WR, &a.gthr[q0 + qq],
                                   sv_w, si_w, a.cap, a.kk, a.kk_final, a.publish_block,
                                   lane);
                }
                thr_r[qb] = fminf(thr_r[qb], thr_w[q]);
            }
        }
    } else {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            float m = VS_INF;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int v = 0; v < 16; ++v) m = fminf(m, acc[qb][rb][v]);
            if (!__ballot(m <= thr_r[qb])) continue;
            const int64_t qg = q0 + qw0 + qb * 32 + l32;
            // row offsets within the wave's tile rows that may be
            // reported: below lim, and above the query (self-join)
            const int omin =
                a.self_join ? (int)max((int64_t)0, min((int64_t)(32 * RB), qg - wr0 + 1)) : 0;
            // one reservation per lane for all of its hits, found as bit
            // masks in VGPRs (no lane mask per value stays live)
            uint32_t mk[RB];
            int c = 0;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                mk[rb] = value_mask16<false>(acc[qb][rb], thr_r[qb]);
                mk[rb] &= rows_below_mask(lim - rb * 32 - 4 * h) &
                          ~rows_below_mask(omin - rb * 32 - 4 * h);
                c += __builtin_popcount(mk[rb]);
            }
            if (c > 0) {
                unsigned long long pos = atomicAdd(a.count, (unsigned long long)c);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        if ((mk[rb] >> v) & 1u) {
                            if (pos < (unsigned long long)a.out_cap) {
                                a.out_q[pos] = (int32_t)qg;
                                a.out_i[pos] = (int32_t)(wr0 + rb * 32 + 8 * (v / 4) + 4 * h + v % 4);
                            }
                            ++pos;
                        }
                    }
            }
        }
    }
}

// Final cut of a top-k scan (MODE 0): every list of this wave's queries
// holds its kk best in slots [0, kk), padded -- one lane per list where kk
// fits in registers, else the lists one after another.  lb0: index of the
// wave's first list bound (its lists' own final thresholds, for the merge's
// verification when lists keep fewer than kk_final).
template <int WR, int BQ, int QB>
__device__ __forceinline__ void gemm_final_cut(const ScanKArgs &a, const EpiCtx &e, int64_t lb0) {
    const int64_t q0 = e.q0;
    const int qw0 = e.qw0, lane = e.lane;
    int *cnt_w = e.cnt_w;
    float *thr = e.thr, *thr_w = e.thr_w, *sv_w = e.sv_w;
    int *si_w = e.si_w;
    float *cv = e.cv;
    int32_t *ci = e.ci;
    wave_sync();
    if (a.kk <= 32) {
        // (64 lists, one per lane, at a time)
        for (int g0 = qw0; g0 < qw0 + 32 * QB; g0 += 64) {
            const int nl = min(64, qw0 + 32 * QB - g0);
            if (a.kk <= 16)
                cut_lists_lanes<16>(cv + (int64_t)g0 * a.cap, ci + (int64_t)g0 * a.cap, cnt_w + g0,
                                    thr_w + g0, thr + g0, nl, WR, &a.gthr[q0 + g0], a.cap, a.kk,
                                    a.kk_final, a.publish_block, a.kk, true, lane, BQ);
            else
                cut_lists_lanes<32>(cv + (int64_t)g0 * a.cap, ci + (int64_t)g0 * a.cap, cnt_w + g0,
                                    thr_w + g0, thr + g0, nl, WR, &a.gthr[q0 + g0], a.cap, a.kk,
                                    a.kk_final, a.publish_block, a.kk, true, lane, BQ);
        }
    } else {
        for (int q = qw0; q < qw0 + 32 * QB; ++q) {
            const int c = cnt_w[q];
            if (c > a.kk) {
                flush_list(cv + (int64_t)q * a.cap, ci + (int64_t)q * a.cap, &cnt_w[q], &thr_w[q],
                           &thr[q], BQ, WR, &a.gthr[q0 + q], sv_w, si_w, a.cap, a.kk, a.kk_final,
                           a.publish_block, lane);
            } else {
                for (int j = c + lane; j < a.kk; j += 64) {
                    cv[(int64_t)q * a.cap + j] = VS_INF;
                    ci[(int64_t)q * a.cap + j] = -1;
                }
            }
        }
    }
    // a list cut to kk < kk_final entries may have dropped rows at or
    // above its own final threshold: the merge checks that value against
    // the query's final kk_final-th value
    if (a.lbound) {
        wave_sync();
        for (int q = qw0 + lane; q < qw0 + 32 * QB; q += 64) a.lbound[lb0 + q] = thr_w[q];
    }
}

// The register-staged kernel writes the next chunk's tiles to LDS between
// the MFMAs of the current chunk's last K-step.
constexpr bool kInterleaveStores = true;
// Row fragments read ahead of the MFMAs that use them in the pipelined chunk
// (two: 4 more VGPRs than one, still spill-free at 256 for top-k).
constexpr int kPipeDist = 2;

template <int ST, int PB, int WR, int WQ, int RB, int QB, int KC, int MODE>
__global__ __launch_bounds__(64 * WR * WQ) void gemm_scan_kernel(ScanKArgs a) {
    using S = GemmShape<ST, PB, WR, WQ, RB, QB, KC>;
    constexpr int NT = S::NT, BR = S::BR, BQ = S::BQ, KP = S::KP;
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x;
    // the wave index in a scalar register: every per-wave base (lists,
    // thresholds, sort buffers) stays scalar instead of taking VGPRs
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int wr = wave % WR, wq = wave / WR;

    int64_t split, qblk;
    if (!map_block_grouped(a.nqblk, a.nsplit, a.qgroup, a.qspc, &split, &qblk)) return;
    int64_t r0 = split * a.rows_per_split;
    const int64_t r1 = min(a.n, r0 + a.rows_per_split);
    const int64_t q0 = qblk * BQ;
    if (MODE == 1 && a.self_join) r0 = max(r0, q0);  // only ids > query
    if (r0 >= r1) return;

    // LDS: two stages, then the lists' counters and thresholds [WR][BQ] and
    // the per-wave sort buffers [NW][cap]
    int *cnt = (int *)(smem + 2 * S::STAGE_BYTES);
    float *thr = (float *)(cnt + WR * BQ);
    float *sv = thr + WR * BQ;
    int *si = (int *)(sv + S::NW * a.cap);
    for (int t = tid; t < WR * BQ; t += NT) {
        cnt[t] = 0;
        thr[t] = q0 + (t % BQ) < a.nq ? VS_INF : -VS_INF;
    }
    int *cnt_w = cnt + wr * BQ;
    float *thr_w = thr + wr * BQ;
    float *sv_w = sv + wave * a.cap;
    int *si_w = si + wave * a.cap;
    const int64_t list_base = ((qblk * a.nsplit + split) * WR + wr) * (int64_t)BQ * a.cap;
    float *cv = MODE == 0 ? a.cand_v + list_base : nullptr;
    int32_t *ci = MODE == 0 ? a.cand_i + list_base : nullptr;
    const int qw0 = wq * 32 * QB;  // the wave's first query in the block
    const EpiCtx ectx{q0, r1, qw0, l32, h, lane, cnt, cnt_w, thr, thr_w, sv_w, si_w, cv, ci};

    float thr_r[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int64_t qg = q0 + qw0 + qb * 32 + l32;
        if (MODE == 0)
            thr_r[qb] = qg < a.nq ? VS_INF : -VS_INF;
        else
            thr_r[qb] = qg < a.nq ? a.athr[qg] : -VS_INF;
    }

    const int nkc = (int)(a.ld / KC);
    const int64_t row_bytes = a.ld * S::ESZ;
    const bool l2 = a.metric == 0;

    // global -> register staging of one K-chunk: A rows, B query planes and
    // (first chunk of a tile) the tile's row norms
    u32x4_t ra[S::A_LOADS], rq[S::B_LOADS];
    f32x4_t rn;
    // physical 16-byte piece of logical piece c of an LDS row r
    auto piece = [](int c, int r) __attribute__((always_inline)) {
        return S::SW ? (c ^ ((r >> 1) & 7)) : c;
    };
    auto lstore_norms = [&](char *stage, int kc) __attribute__((always_inline)) {
        if (kc == 0 && l2 && tid < BR / 4)
            *(f32x4_t *)((float *)((uint16_t *)stage + S::STAGE_ELEMS) + 4 * tid) = rn;
    };
    // piece p of a chunk: A load p (p < A_LOADS; piece 0 also carries a
    // tile's row norms) or B load p - A_LOADS.  Buffer loads:
    // a thread's pieces sit at one 32-bit offset from a per-chunk resource
    // plus a uniform step per piece, so they need one address VGPR per
    // operand; LDS writes likewise step by whole 16-row groups (the swizzle
    // repeats every 16 rows), one base address per operand.
    constexpr int NLD = S::A_LOADS + S::B_LOADS;
    constexpr int A_STEP = NT / S::A_CPR;       // rows per A piece
    constexpr int B_STEP = NT / S::B_CPR / PB;  // queries per B piece
    static_assert(NT % S::A_CPR == 0 && A_STEP % 16 == 0 && NT % (S::B_CPR * PB) == 0 &&
                      B_STEP % 16 == 0,
                  "a thread's pieces are whole 16-row groups apart");
    const int a_row = tid / S::A_CPR, a_c = tid % S::A_CPR;
    const int b_row = tid / S::B_CPR, b_c = tid % S::B_CPR;  // b_row: q PB + plane
    const int a_voff = a_row * (int)row_bytes + a_c * 16;
    // prepared queries keep two plane rows of ld elements per query
    const int b_voff = ((b_row / PB) * 2 + b_row % PB) * (int)a.ld * 2 + b_c * 16;
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.qp + q0 * 2 * a.ld), 0, (int)min((int64_t)INT32_MAX, (int64_t)BQ * 4 * a.ld),
        kBufRsrcWord3);
    // LDS element offsets of the thread's first A and B piece
    int a_soff, b_soff;
    if constexpr (ST == 1) {
        a_soff = a_row * KP + piece(a_c, a_row) * 8;
    } else {
        a_soff = a_row * KP + piece(a_c >> 1, a_row) * 8 + (a_c & 1) * 4;
    }
    {
        const int q = b_row / PB, pl = b_row % PB;
        b_soff = (pl * BQ + q) * KP + piece(b_c, q) * 8;
    }
    auto load_piece = [&](int p, int64_t trow, int kc, bool norms = true) __attribute__((always_inline)) {
        if (p < S::A_LOADS) {
            // the last tile reads at most BR rows past the end, inside the
            // allocation's slack rows; the resource stops there
            const int64_t lim = min((int64_t)INT32_MAX, (a.n - trow + BR) * row_bytes);
            const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)((const char *)a.xb + trow * row_bytes), 0, (int)lim, kBufRsrcWord3);
            ra[p] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             xrs, a_voff, p * A_STEP * (int)row_bytes + kc * KC * S::ESZ, 0));
            if (p == 0 && kc == 0 && l2 && norms && tid < BR / 4)
                rn = *(const f32x4_t *)(a.xn + trow + 4 * tid);
        } else {
            const int j = p - S::A_LOADS;
            rq[j] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             qrs, b_voff, j * B_STEP * (int)a.ld * 4 + kc * KC * 2, 0));
        }
    };
    auto store_piece = [&](int p, char *stage, int kc) __attribute__((always_inline)) {
        uint16_t *As = (uint16_t *)stage;
        uint16_t *Bs = As + S::AP * BR * KP;
        if (p < S::A_LOADS) {
            uint16_t *dst = As + a_soff + p * A_STEP * KP;
            if constexpr (ST == 1) {
                *(u32x4_t *)dst = ra[p];
            } else {
                typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
                const f32x4_t f = __builtin_bit_cast(f32x4_t, ra[p]);
                const bf16x4_t hi = __builtin_convertvector(f, bf16x4_t);
                *(u32x2_t *)dst = __builtin_bit_cast(u32x2_t, hi);
                if constexpr (ST == 0) {
                    const bf16x4_t lo =
                        __builtin_convertvector(f - __builtin_convertvector(hi, f32x4_t), bf16x4_t);
                    *(u32x2_t *)(dst + BR * KP) = __builtin_bit_cast(u32x2_t, lo);
                }
            }
            if (p == 0) lstore_norms(stage, kc);
        } else {
            const int j = p - S::A_LOADS;
            *(u32x4_t *)(Bs + b_soff + j * B_STEP * KP) = rq[j];
        }
    };

    f32x16_t acc[QB][RB];
    uint32_t gt[QB];

    // One K-chunk of MFMAs from LDS stage `stage`; with `nstage`, the next
    // chunk's A and B tiles (already loaded into registers) are written to
    // that stage between the MFMAs of the last K-step, so that the LDS
    // writes overlap the matrix pipe instead of following it.  first_c: 0 a
    // later chunk; 1 a tile's first chunk, whose first K-step takes the row
    // norms (L2) or zero (IP) as its C operand; 2 a tile's first chunk of an
    // inner-product scan (zero C operand, no metric test inside).  ld(p)
    // issues the next chunk's load p.
    auto compute = [&](const char *stage, auto first_c, char *nstage, auto ld) __attribute__((always_inline)) {
        constexpr int FM = decltype(first_c)::value;
        constexpr bool FIRST = FM != 0;
        constexpr bool IL = kInterleaveStores;
        const uint16_t *As = (const uint16_t *)stage;
        const uint16_t *Bs = As + S::AP * BR * KP;
        // the lane's A and B rows (rows wr 32 RB + l32 + 32 rb and
        // qw0 + l32 + 32 qb, offsets of whole 32-row blocks from l32, so all
        // swizzled as row l32); K-step ks reads
        // logical piece 2 ks + h of them
        const uint16_t *al_ = As + (wr * 32 * RB + l32) * KP;
        const uint16_t *bl_ = Bs + (qw0 + l32) * KP;
        auto koff = [&](int ks) __attribute__((always_inline)) { return piece(2 * ks + h, l32) * 8; };
        const float *Ns = (const float *)(As + S::STAGE_ELEMS) + wr * 32 * RB + 4 * h;
        if constexpr (ST == 1 && PB == 1 && FM != 1 && IL) {
            // Software-pipelined chunk (bf16 rows, one query plane): the
            // (K-step, row block) pairs run in order; the row fragment of the
            // pair kPipeDist ahead, and at a K-step's first row block the next
            // K-step's query fragments, are read before this pair's MFMAs, so
            // the matrix pipe waits on no fragment read issued just before it.
            // The next chunk's global loads follow the MFMAs of K-step 0's
            // pairs, and its LDS writes (into the stage last read before the
            // previous barrier) the MFMAs of the pairs of the last SK K-steps,
            // spread evenly: no pair carries a burst of memory instructions,
            // and the loads have most of the chunk to arrive.
            constexpr int NKS = KC / 16, NI = NKS * RB;
            constexpr int NST = S::A_LOADS + S::B_LOADS;
            constexpr int PD = kPipeDist;
            constexpr int SK = MODE == 1 ? 3 : 2;  // (measured best per mode)
            constexpr int SP = SK * RB < NI ? SK * RB : NI;  // pairs that carry the writes
            auto ld_lo = [](int rb) __attribute__((always_inline)) { return rb * NLD / RB; };
            auto st_lo = [](int j) __attribute__((always_inline)) { return j * NST / SP; };
            bf16x8_t af[PD + 1], bq[2][QB];
            auto rd_a = [&](int i) __attribute__((always_inline)) {
                return __builtin_bit_cast(
                    bf16x8_t, *(const u32x4_t *)(al_ + (i % RB) * 32 * KP + koff(i / RB)));
            };
            auto rd_b = [&](int ks, int qb) __attribute__((always_inline)) {
                return __builtin_bit_cast(bf16x8_t,
                                          *(const u32x4_t *)(bl_ + qb * 32 * KP + koff(ks)));
            };
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) bq[0][qb] = rd_b(0, qb);
#pragma unroll
            for (int i = 0; i < PD; ++i) af[i] = rd_a(i);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int ks = i / RB, rb = i % RB;
                if (i + PD < NI) af[(i + PD) % (PD + 1)] = rd_a(i + PD);
                if (rb == 0 && ks + 1 < NKS) {
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) bq[(ks + 1) & 1][qb] = rd_b(ks + 1, qb);
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    acc[qb][rb] = mfma32_bf16(af[i % (PD + 1)], bq[ks & 1][qb],
                                              FM == 2 && ks == 0 ? f32x16_t{} : acc[qb][rb]);
                if (ks == 0) {
#pragma unroll
                    for (int p = ld_lo(rb); p < ld_lo(rb + 1); ++p) ld(p);
                }
                // (the writes stay in program order after the fragment reads
                // before them: the compiler cannot tell the two stages apart)
                if (i >= NI - SP) {
#pragma unroll
                    for (int p = st_lo(i - (NI - SP)); p < st_lo(i - (NI - SP) + 1); ++p)
                        store_piece(p, nstage, -1);
                }
            }
            // the order: the first reads, then per pair its look-ahead reads,
            // its MFMAs, its loads (K-step 0) and its writes (last SK K-steps)
            __builtin_amdgcn_sched_group_barrier(0x100, QB + PD, 0);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int ks = i / RB, rb = i % RB;
                if (i + PD < NI) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                if (rb == 0 && ks + 1 < NKS) __builtin_amdgcn_sched_group_barrier(0x100, QB, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
                if (ks == 0) {
#pragma unroll
                    for (int p = ld_lo(rb); p < ld_lo(rb + 1); ++p)
                        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
                if (i >= NI - SP) {
#pragma unroll
                    for (int p = st_lo(i - (NI - SP)); p < st_lo(i - (NI - SP) + 1); ++p)
                        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                }
            }
            return;
        }
#pragma unroll
        for (int p = 0; p < NLD; ++p) ld(p);
#pragma unroll
        for (int ks = 0; ks < KC / 16; ++ks) {
            // the last K-step and the stores form a scheduling region of
            // their own (the group barriers below order it)
            if (IL && ks + 1 == KC / 16) __builtin_amdgcn_sched_barrier(0);
            bf16x8_t b0[QB], b1[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                b0[qb] = __builtin_bit_cast(bf16x8_t,
                                            *(const u32x4_t *)(bl_ + qb * 32 * KP + koff(ks)));
                if constexpr (PB == 2)
                    b1[qb] = __builtin_bit_cast(
                        bf16x8_t, *(const u32x4_t *)(bl_ + BQ * KP + qb * 32 * KP + koff(ks)));
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const bf16x8_t ah = __builtin_bit_cast(
                    bf16x8_t, *(const u32x4_t *)(al_ + rb * 32 * KP + koff(ks)));
                bf16x8_t alo;
                if constexpr (ST == 0)
                    alo = __builtin_bit_cast(
                        bf16x8_t, *(const u32x4_t *)(al_ + BR * KP + rb * 32 * KP + koff(ks)));
                f32x16_t x16;
                if (FIRST && ks == 0) {
                    if (l2) {
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const f32x4_t q4 = *(const f32x4_t *)(Ns + rb * 32 + 8 * u);
#pragma unroll
                            for (int e = 0; e < 4; ++e) x16[4 * u + e] = q4[e];
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 16; ++e) x16[e] = 0.f;
                    }
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    acc[qb][rb] = mfma32_bf16(ah, b0[qb], (FIRST && ks == 0) ? x16 : acc[qb][rb]);
                    if constexpr (ST == 0) acc[qb][rb] = mfma32_bf16(alo, b0[qb], acc[qb][rb]);
                    if constexpr (PB == 2) acc[qb][rb] = mfma32_bf16(ah, b1[qb], acc[qb][rb]);
                }
            }
        }
        if constexpr (IL) {
#pragma unroll
            for (int p = 0; p < NLD; ++p) store_piece(p, nstage, -1);
            // schedule of the last K-step: its B fragment reads, then per
            // row block its A fragment read(s), its MFMAs and one store of
            // the next stage; the remaining stores last
            constexpr int MPB = QB * (1 + (ST == 0) + (PB == 2));  // MFMAs per row block
            constexpr int NST = S::A_LOADS * (ST == 0 ? 2 : 1) + S::B_LOADS;
            __builtin_amdgcn_sched_group_barrier(0x100, QB * PB, 0);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                __builtin_amdgcn_sched_group_barrier(0x100, ST == 0 ? 2 : 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, MPB, 0);
                if (rb < NST) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            }
            if (NST > RB) __builtin_amdgcn_sched_group_barrier(0x200, NST > RB ? NST - RB : 0, 0);
        }
    };

#pragma unroll
    for (int p = 0; p < NLD; ++p) load_piece(p, r0, 0);
#pragma unroll
    for (int p = 0; p < NLD; ++p) store_piece(p, smem, 0);
    __syncthreads();

    int par = 0;  // stage holding the current chunk
    // the first tile seeds the lists' thresholds when two lanes can hold kk
    // values (ceil(kk / 2) <= 16 * RB)
    bool seeded = (a.kk + 1) / 2 > 16 * RB;
    for (int64_t t0 = r0; t0 < r1; t0 += BR) {
        const bool last_tile = t0 + BR >= r1;
        // the epilogue stays after the K loop: values it computes from the
        // tile alone (row ids, offset masks) are then not hoisted into
        // registers held across the loop
        for (int kc = 0; kc < nkc; ++kc) {
            char *cur = smem + par * S::STAGE_BYTES;
            char *nxt = smem + (par ^ 1) * S::STAGE_BYTES;
            const bool last_chunk = kc + 1 == nkc;
            const bool more = !(last_chunk && last_tile);
            const int kc_next = last_chunk ? 0 : kc + 1;
            const int64_t t_next = last_chunk ? t0 + BR : t0;
            // the next chunk's loads, issued inside compute: unconditionally
            // (past the last tile they read slack rows), the norms only when a
            // next tile follows
            auto ld = [&](int p) __attribute__((always_inline)) {
                load_piece(p, t_next, kc_next, more);
            };
            if (kc == 0) {
                if constexpr (MODE == 0) {
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
                        gt[qb] = __hip_atomic_load(&a.gthr[q0 + qw0 + qb * 32 + l32],
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (l2)
                    compute(cur, std::integral_constant<int, 1>{}, nxt, ld);
                else
                    compute(cur, std::integral_constant<int, 2>{}, nxt, ld);
            } else {
                compute(cur, std::integral_constant<int, 0>{}, nxt, ld);
            }
            // (with interleaved stores, the last chunk stores stale registers
            // into the free stage, which nothing reads afterwards)
            if (!kInterleaveStores && more) {
#pragma unroll
                for (int p = 0; p < NLD; ++p) store_piece(p, nxt, -1);
            }
            if (more) lstore_norms(nxt, kc_next);
            par ^= 1;
            if (!last_chunk) __syncthreads();
        }
        gemm_epilogue<WR, BQ, RB, QB, MODE>(acc, a, ectx, t0 + wr * 32 * RB, thr_r, gt, seeded);
        __syncthreads();
    }

    if constexpr (MODE == 0)
        gemm_final_cut<WR, BQ, QB>(a, ectx, ((qblk * a.nsplit + split) * WR + wr) * (int64_t)BQ);
}

// ---------------------------------------------------------------------------
// Four-wave pipelined GEMM-tiled scan (option gemm4): bf16 rows, one query
// plane (configs[2] at large batches; the self-join's bf16 copy of the rows).
//
// 256 rows x 256 queries per tile.  Wave (wr, wq) multiplies rows
// wr*128 .. +128 by queries wq*128 .. +128 with sixteen 32 x 32 accumulator
// blocks (256 accumulation registers), one wave per SIMD: per 16-element
// K-step 4 row and 4 query fragment reads feed 16 MFMAs (0.5 reads per MFMA,
// against 0.75 in the eight-wave kernel).
//
// K-chunks of 32 elements cycle through four LDS stages (chunk g in stage
// g % 4; rows and query planes 64 bytes each, 16-byte pieces XOR-swizzled by
// (row >> 2) & 3, so the 16 lanes of a fragment read hit 16 distinct 16-byte
// bank groups of the 64-bank LDS, and so do the row writes).  During chunk g:
//   - the global loads of chunk g + 3 are issued (into the staging set that
//     chunk g + 1 left free), one after every second MFMA of K-step 0, while
//     K-step 1's fragments are read, one after each other MFMA;
//   - chunk g + 2 (loaded during chunk g - 1) is written to its stage, whose
//     last reader, chunk g - 2, finished before the previous barrier, and the
//     fragments of chunk g + 1's K-step 0 -- written during chunk g - 1, so
//     visible since the previous barrier -- are read, both during the first
//     half of K-step 1's MFMAs;
//   - one barrier.
// So the matrix pipe never waits on a fragment read issued after a barrier,
// and a global load has about one and a half chunks to arrive.  Loads are
// issued unconditionally (past the end they read slack rows or nothing), so
// the waits before the LDS writes leave the younger loads in flight.  A
// tile's first chunk sits in stage 0 (ld is a multiple of 128 elements for
// bf16 rows, so a tile has a multiple of four chunks), which also carries
// the tile's row norms (L2).  The epilogue (lists, thresholds, range
// appends) is the shared gemm_epilogue, once per tile.
// ---------------------------------------------------------------------------
namespace g4 {
constexpr int NW = 4, NT = 256, WR = 2, WQ = 2, RB = 4, QB = 4, BR = 256, BQ = 256;
constexpr int KC = 32, NSTG = 4;
constexpr int ROWB = KC * 2;                 // bytes per row (query) per chunk
constexpr int A_OFF = 0, B_OFF = BR * ROWB;  // within a stage
constexpr int N_OFF = B_OFF + BQ * ROWB;     // row norms of the tile (stage 0, L2)
constexpr int STAGE = N_OFF + BR * 4;
static_assert(NW == WR * WQ && NT == 64 * NW && BR == WR * 128 && BQ == WQ * 128,
              "each wave multiplies 128 rows by 128 queries");
constexpr int LOADS = BR * (ROWB / 16) / NT;  // 16-byte loads per thread and operand
static_assert(LOADS == 4 && BQ == BR, "thread layout of the loads");
static_assert(2 * LOADS == RB + QB && RB * QB == 4 * LOADS,
              "per K-step: one load (or LDS write) and one fragment read per two MFMAs");
static_assert(BR <= kRowSlack, "the last row tile reads at most kRowSlack rows past the end");
}  // namespace g4

size_t gemm4_lds_bytes(int cap) {
    return (size_t)g4::NSTG * g4::STAGE + (size_t)g4::WR * g4::BQ * 8 + (size_t)g4::NW * cap * 8;
}

template <int MODE, bool L2>
__global__ __launch_bounds__(256) void gemm4_scan_kernel(ScanKArgs a) {
    using namespace g4;
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x;
    // the wave index in a scalar register: every per-wave base (lists,
    // thresholds, sort buffers) stays scalar instead of taking VGPRs
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int wr = wave % WR, wq = wave / WR;

    int64_t split, qblk;
    if (!map_block_grouped(a.nqblk, a.nsplit, a.qgroup, a.qspc, &split, &qblk)) return;
    int64_t r0 = split * a.rows_per_split;
    const int64_t r1 = min(a.n, r0 + a.rows_per_split);
    const int64_t q0 = qblk * BQ;
    if (MODE == 1 && a.self_join) r0 = max(r0, q0);  // only ids > query
    if (r0 >= r1) return;

    // LDS: four stages, then the lists' counters and thresholds [WR][BQ] and
    // the per-wave sort buffers [NW][cap]
    int *cnt = (int *)(smem + NSTG * STAGE);
    float *thr = (float *)(cnt + WR * BQ);
    float *sv = thr + WR * BQ;
    int *si = (int *)(sv + NW * a.cap);
    for (int t = tid; t < WR * BQ; t += NT) {
        cnt[t] = 0;
        thr[t] = q0 + (t % BQ) < a.nq ? VS_INF : -VS_INF;
    }
    int *cnt_w = cnt + wr * BQ;
    float *thr_w = thr + wr * BQ;
    const int64_t list_base = ((qblk * a.nsplit + split) * WR + wr) * (int64_t)BQ * a.cap;
    float *cv = MODE == 0 ? a.cand_v + list_base : nullptr;
    int32_t *ci = MODE == 0 ? a.cand_i + list_base : nullptr;
    const int qw0 = wq * 32 * QB;
    const EpiCtx ectx{q0, r1, qw0, l32, h, lane, cnt, cnt_w, thr, thr_w,
                      sv + wave * a.cap, si + wave * a.cap, cv, ci};

    float thr_r[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int64_t qg = q0 + qw0 + qb * 32 + l32;
        if (MODE == 0)
            thr_r[qb] = qg < a.nq ? VS_INF : -VS_INF;
        else
            thr_r[qb] = qg < a.nq ? a.athr[qg] : -VS_INF;
    }

    const int nkc = (int)(a.ld / KC);  // a multiple of 4
    const int row_bytes = (int)(a.ld * 2);

    // ---- global -> staging registers: thread t loads rows (queries)
    // t / 4 + 64 i, 16-byte piece t % 4 of the chunk ----
    const int ld_row = tid >> 2, ld_pc = tid & 3;
    const int ld_voff_a = ld_row * row_bytes + ld_pc * 16;
    const int ld_voff_b = ld_row * (row_bytes * 2) + ld_pc * 16;  // two planes per query
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.qp + q0 * 2 * a.ld), 0, (int)min((int64_t)INT32_MAX, (int64_t)BQ * 4 * a.ld),
        kBufRsrcWord3);
    // LDS byte offset (within a stage) of the thread's writes: row ld_row +
    // 64 i, physical piece ld_pc ^ ((row >> 2) & 3) (64 i keeps the swizzle)
    const int st_off = ld_row * ROWB + ((ld_pc ^ ((ld_row >> 2) & 3)) << 4);

    u32x4_t sa[2][LOADS], sb[2][LOADS];
    float sn;  // one row norm per thread (row tid of a tile)

    // Every chunk's loads are issued unconditionally -- past the last chunk
    // they read rows beyond the split end (inside the allocation's slack) or
    // nothing at all (the resource's record count is zero) -- so the waits
    // before the LDS writes count only the loads issued since (a skipped
    // load would make every wait a full drain).
    // buffer resources of a tile's rows and row norms: the last tile reads
    // at most BR rows past the end, inside the allocation's slack rows
    auto rows_rs = [&](int64_t trow) __attribute__((always_inline)) {
        const int64_t lim =
            min((int64_t)INT32_MAX, max((int64_t)0, (a.n - trow + BR) * (int64_t)row_bytes));
        return __builtin_amdgcn_make_buffer_rsrc((void *)((const char *)a.xb + trow * row_bytes), 0,
                                                 (int)lim, kBufRsrcWord3);
    };
    auto norms_rs = [&](int64_t trow) __attribute__((always_inline)) {
        const int64_t lim = min((int64_t)INT32_MAX, max((int64_t)0, (a.n - trow + BR) * 4));
        return __builtin_amdgcn_make_buffer_rsrc((void *)(a.xn + trow), 0, (int)lim, kBufRsrcWord3);
    };
    auto issue = [&](auto set_c, __amdgpu_buffer_rsrc_t xrs, int kc) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            sa[S][i] = buf_load16(xrs, ld_voff_a, i * 64 * row_bytes + kc * ROWB);
            sb[S][i] = buf_load16(qrs, ld_voff_b, i * 64 * row_bytes * 2 + kc * ROWB);
        }
    };
    // the row norms of a tile: thread t loads row t
    auto issue_norms = [&](__amdgpu_buffer_rsrc_t nrs) __attribute__((always_inline)) {
        if constexpr (L2)
            sn = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(nrs, tid * 4, 0, 0));
    };
    auto write = [&](auto set_c, auto stage_c) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value, T = decltype(stage_c)::value;
        char *st = smem + T * STAGE;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            *(u32x4_t *)(st + A_OFF + st_off + i * 64 * ROWB) = sa[S][i];
            *(u32x4_t *)(st + B_OFF + st_off + i * 64 * ROWB) = sb[S][i];
        }
    };
    auto write_norms = [&]() __attribute__((always_inline)) {
        if constexpr (L2) *(float *)(smem + N_OFF + 4 * tid) = sn;
    };

    // ---- fragments: lane (l32, h) reads row wr*128 + 32 rb + l32 and query
    // qw0 + 32 qb + l32, logical piece 2 ks + h of the chunk ----
    const int swz = (l32 >> 2) & 3;
    const int fa0 = (wr * 128 + l32) * ROWB + (((0 + h) ^ swz) << 4);
    const int fa1 = (wr * 128 + l32) * ROWB + (((2 + h) ^ swz) << 4);
    const int fb0 = B_OFF + (qw0 + l32) * ROWB + (((0 + h) ^ swz) << 4);
    const int fb1 = B_OFF + (qw0 + l32) * ROWB + (((2 + h) ^ swz) << 4);
    bf16x8_t fa[2][RB], fb[2][QB];
    auto read_frags = [&](auto buf_c, auto stage_c, auto ks_c) __attribute__((always_inline)) {
        constexpr int F = decltype(buf_c)::value, T = decltype(stage_c)::value;
        constexpr int KS = decltype(ks_c)::value;
        const char *st = smem + T * STAGE;
        const int oa = KS == 0 ? fa0 : fa1, ob = KS == 0 ? fb0 : fb1;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
            fa[F][rb] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(st + oa + rb * 32 * ROWB));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
            fb[F][qb] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(st + ob + qb * 32 * ROWB));
    };

    f32x16_t acc[QB][RB];
    uint32_t gt[QB];

    // 16 MFMAs of one K-step from fragment buffer F; FIRST: the tile's first
    // K-step, whose C operand is the row norms (L2) or zero (IP)
    auto mfmas = [&](auto buf_c, auto first_c) __attribute__((always_inline)) {
        constexpr int F = decltype(buf_c)::value;
        constexpr bool FIRST = decltype(first_c)::value;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            f32x16_t c0;
            if constexpr (FIRST) {
                if constexpr (L2) {
                    const float *Ns = (const float *)(smem + N_OFF) + wr * 128 + rb * 32 + 4 * h;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f32x4_t q4 = *(const f32x4_t *)(Ns + 8 * u);
#pragma unroll
                        for (int e = 0; e < 4; ++e) c0[4 * u + e] = q4[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 16; ++e) c0[e] = 0.f;
                }
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
                acc[qb][rb] = mfma32_bf16(fa[F][rb], fb[F][qb], FIRST ? c0 : acc[qb][rb]);
        }
    };

    // Chunks go in groups of four, g0 .. g0 + 3 (a group never spans two
    // tiles); kc_c is the current group's first K-chunk and xrs_c its tile's
    // row resource, kc_n / xrs_n / nrs_n the next group's.  Chunk g0 + T
    // (stage T, staging set S = T & 1 for chunk g0 + T + 2) issues the loads
    // of chunk g0 + T + 3, and at T = 1 the norms of the next group's tile
    // (written with that group's first chunk at T = 2: unchanged unless it
    // starts a tile, and the current tile's were used by its first chunk).
    // The next group's positions and resources are computed at the end of
    // the group's last chunk, before its barrier, where the wave waits
    // anyway (not between a barrier and the MFMAs after it).
    int64_t trow_n = r0;
    int kc_c = 0, kc_n = 0;
    __amdgpu_buffer_rsrc_t xrs_c = rows_rs(r0), xrs_n, nrs_n;
    auto advance = [&]() __attribute__((always_inline)) {
        trow_n = kc_n + 4 == nkc ? trow_n + BR : trow_n;
        kc_n = kc_n + 4 == nkc ? 0 : kc_n + 4;
        xrs_n = rows_rs(trow_n);
        nrs_n = norms_rs(trow_n);
    };
    advance();  // the second group's
    auto chunk = [&](auto stage_c, auto first_c) __attribute__((always_inline)) {
        constexpr int T = decltype(stage_c)::value;
        constexpr int S = T & 1;
        if constexpr (T == 0)
            issue(std::integral_constant<int, S ^ 1>{}, xrs_c, kc_c + 3);
        else
            issue(std::integral_constant<int, S ^ 1>{}, xrs_n, kc_n + T - 1);
        if constexpr (T == 1) issue_norms(nrs_n);
        // K-step 0 from fa/fb[0] while K-step 1's fragments are read; one
        // global load and one fragment read after every second MFMA
        read_frags(std::integral_constant<int, 1>{}, stage_c, std::integral_constant<int, 1>{});
        mfmas(std::integral_constant<int, 0>{}, first_c);
#pragma unroll
        for (int i = 0; i < 2 * LOADS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // fragment read
        }
        if (T == 1 && L2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        // chunk g0 + T + 2 into its stage and the next chunk's K-step 0
        // fragments read: one LDS write and one read after each of the
        // first eight MFMAs of K-step 1, so the last eight leave them time
        // to complete before the barrier waits for them
        write(std::integral_constant<int, S>{}, std::integral_constant<int, (T + 2) & 3>{});
        if constexpr (T == 2) write_norms();
        read_frags(std::integral_constant<int, 0>{}, std::integral_constant<int, (T + 1) & 3>{},
                   std::integral_constant<int, 0>{});
        mfmas(std::integral_constant<int, 1>{}, std::false_type{});
        if (T == 2 && L2) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
#pragma unroll
        for (int i = 0; i < 2 * LOADS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // fragment read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, RB * QB - 2 * LOADS, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (T == 3) {
            xrs_c = xrs_n;
            kc_c = kc_n;
            advance();
        }
        __syncthreads();
    };
    // one group of four chunks; FIRST: the tile's first group
    auto group = [&](auto first_c) __attribute__((always_inline)) {
        chunk(std::integral_constant<int, 0>{}, first_c);
        chunk(std::integral_constant<int, 1>{}, std::false_type{});
        chunk(std::integral_constant<int, 2>{}, std::false_type{});
        chunk(std::integral_constant<int, 3>{}, std::false_type{});
    };

    // prologue: chunks 0 and 1 (and the first tile's norms) into stages 0
    // and 1 from sets 0 and 1, chunk 2's loads issued into set 0, the first
    // fragments read
    issue(std::integral_constant<int, 0>{}, xrs_c, 0);
    issue(std::integral_constant<int, 1>{}, xrs_c, 1);
    issue_norms(norms_rs(r0));
    write(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    write(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    write_norms();
    issue(std::integral_constant<int, 0>{}, xrs_c, 2);
    __syncthreads();
    read_frags(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{},
               std::integral_constant<int, 0>{});

    // the first tile seeds the lists' thresholds when two lanes can hold kk
    // values (ceil(kk / 2) <= 16 * RB)
    bool seeded = (a.kk + 1) / 2 > 16 * RB;
    for (int64_t t0 = r0; t0 < r1; t0 += BR) {
        if constexpr (MODE == 0) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
                gt[qb] = __hip_atomic_load(&a.gthr[q0 + qw0 + qb * 32 + l32], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        }
        group(std::true_type{});
        for (int kc = 4; kc < nkc; kc += 4) group(std::false_type{});
        gemm_epilogue<WR, BQ, RB, QB, MODE>(acc, a, ectx, t0 + wr * 128, thr_r, gt, seeded);
        __syncthreads();
    }

    if constexpr (MODE == 0)
        gemm_final_cut<WR, BQ, QB>(a, ectx, ((qblk * a.nsplit + split) * WR + wr) * (int64_t)BQ);
}

template <int MODE>
hipError_t launch_gemm_scan(int storage, int planes, const ScanPlan &plan, const ScanKArgs &args,
                            hipStream_t st) {
    const int64_t grid = tile_grid_space(plan.nqblk, plan.nsplit, plan.tile_group, plan.tile_spc);
    ScanKArgs ga = args;
    ga.qgroup = plan.tile_group;
    ga.qspc = plan.tile_spc;
    ga.publish_block = plan.lw * plan.kk >= plan.kk_final;
    // cut lists at twice their keep: each cut tightens the list's threshold
    // for the price of one sort of ~2 kk entries
    ga.flush_at = std::max(2 * plan.kk, 16);
    void (*fn)(ScanKArgs) = nullptr;
    if (plan.g_pipe) {
        // the four-wave pipelined kernel: bf16 rows, one query plane, rows
        // of whole four-chunk groups
        if (storage != 1 || planes != 1 || args.ld % (4 * g4::KC) != 0 || plan.lw != g4::WR ||
            plan.bn != g4::BQ || plan.tile_rb != g4::RB || plan.g_qb != g4::QB)
            return hipErrorInvalidValue;
        fn = args.metric == 0 ? gemm4_scan_kernel<MODE, true> : gemm4_scan_kernel<MODE, false>;
        const size_t lds = plan.lds_bytes;
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(g4::NT), lds, st, ga);
        return hipGetLastError();
    }
#define VS_GPICK(ST_, PB_, WR_, WQ_, RB_, QB_, KC_)                                            \
    if (storage == ST_ && planes == PB_ && plan.lw == WR_ && plan.g_wq == WQ_ &&                 \
        plan.tile_rb == RB_ && plan.g_qb == QB_ && plan.tile_kc == KC_)                          \
        fn = gemm_scan_kernel<ST_, PB_, WR_, WQ_, RB_, QB_, KC_, MODE>;
    VS_GEMM_SHAPES(VS_GPICK)
#undef VS_GPICK
    if (!fn) return hipErrorInvalidValue;
    const size_t lds = plan.lds_bytes;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(64 * plan.lw * plan.g_wq), lds, st, ga);
    return hipGetLastError();
}

template hipError_t launch_gemm_scan<0>(int, int, const ScanPlan &, const ScanKArgs &, hipStream_t);
template hipError_t launch_gemm_scan<1>(int, int, const ScanPlan &, const ScanKArgs &, hipStream_t);

}  // namespace vs
