// vs_tile.hip -- the tiled distance scan of libvs_hip.so for large query
// batches (gfx950).
//
// One workgroup of NW waves owns a block of BQ = 32*QB queries and one split
// of the database rows, which it walks in row tiles of NW x WR rows (WR =
// 32*RB rows per wave).  Each wave multiplies its own WR rows by all BQ
// queries with v_mfma_f32_32x32x16_bf16 (on gfx950 it sustains about 2.1
// PFLOP/s at one wave per SIMD, over twice the 16x16x32 form), holding
// QB x RB accumulator blocks of 32 x 32:
//   - the block's prepared query planes (the B operand) are copied into LDS
//     once and stay there, so the main loop needs no barrier and the L2 only
//     carries database rows;
//   - database rows go HBM -> registers straight into the MFMA A-operand
//     layout (lane (r, h) of a 32-row block holds row r, K elements
//     8h .. 8h+7 of each 16-wide K-step), with the next K-chunk's loads in
//     flight while the current one is multiplied; they never touch LDS.
// Every database byte a wave loads feeds BQ queries, every query byte it
// reads from LDS feeds WR rows.
//
// Operands (the convention of the streaming scan in vs_kernels.hip): the
// prepared queries hold bf16 planes of s*q (s = -2 for L2, -1 for IP) and the
// accumulator starts at xn (L2) or 0 (IP), so it is "smaller is better" for
// both metrics.  fp32 rows are split in registers into bf16 hi and lo; the
// products are hi*q0 + lo*q0 (+ hi*q1 when the queries need a second plane).
//
// Epilogue per row tile: the same per-(wave, query) candidate lists, list
// flushes, per-query shared thresholds (MODE 0) and range appends (MODE 1) as
// the streaming scan, so the merge, re-rank, k-means and range kernels read
// its output unchanged.  The full distance matrix is never written.
#include <limits.h>

#include <type_traits>

#include "vs_device.h"

namespace vs {

size_t tile_lds_bytes(int qb, int pb, int nw, int cap, int64_t ld) {
    const size_t bq = (size_t)32 * qb;
    return (size_t)pb * bq * (size_t)(ld + 8) * 2 + (size_t)nw * bq * 8 + (size_t)nw * cap * 8;
}

// Register fragment of one 32-row block and one 16-wide K-step: 8 bf16 (one
// 16-byte load) for bf16 rows, 8 fp32 (two loads) for fp32 rows.
template <int ST>
struct ARows {
    static constexpr int W = ST == 0 ? 2 : 1;
};

template <int ST>
__device__ __forceinline__ void a_split(const u32x4_t (&v)[ARows<ST>::W], bf16x8_t &hi,
                                        bf16x8_t &lo) {
    if constexpr (ST == 1) {
        hi = __builtin_bit_cast(bf16x8_t, v[0]);
    } else {
        typedef float f32x8_t __attribute__((ext_vector_type(8)));
        const f32x8_t f = __builtin_bit_cast(f32x8_t, v);
        hi = __builtin_convertvector(f, bf16x8_t);
        lo = __builtin_convertvector(f - __builtin_convertvector(hi, f32x8_t), bf16x8_t);
    }
}

// Issues the loads of one K-chunk (kc) of the wave's WR rows starting at row
// offset `roff` from the lane's base `arow` (row l % 32, K offset 8 * (l / 32))
// into `dst`.
template <int ST, int RB, int KC>
__device__ __forceinline__ void a_load(u32x4_t (&dst)[KC / 16][RB][ARows<ST>::W], const char *arow,
                                       int64_t row_bytes, int64_t roff, int kc) {
    constexpr int ESZ = ST == 0 ? 4 : 2;
    const char *p = arow + roff * row_bytes + (int64_t)kc * KC * ESZ;
#pragma unroll
    for (int ks = 0; ks < KC / 16; ++ks)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int h = 0; h < ARows<ST>::W; ++h)
                dst[ks][rb][h] = *(const u32x4_t *)(p + rb * 32 * row_bytes + ks * 16 * ESZ + h * 16);
}

// One K-chunk of MFMAs: the wave's rows (registers) times all BQ queries
// (LDS, row stride bs elements, plane 1 at +bplane; bw = this lane's query
// row l % 32 at the chunk's K offset + 8 * (l / 32)).  FIRST: the tile's
// first chunk, whose first K-step takes the accumulator's start value x16 as
// its C operand.
template <int ST, int PB, int QB, int RB, int KC, bool FIRST>
__device__ __forceinline__ void tile_mma(f32x16_t (&acc)[QB][RB], const f32x16_t (&x16)[RB],
                                         const u32x4_t (&a)[KC / 16][RB][ARows<ST>::W],
                                         const uint16_t *bw, int bs, int bplane) {
#pragma unroll
    for (int ks = 0; ks < KC / 16; ++ks) {
        bf16x8_t ah[RB], al[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) a_split<ST>(a[ks][rb], ah[rb], al[rb]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const bf16x8_t b0 =
                __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(bw + qb * 32 * bs + ks * 16));
            bf16x8_t b1;
            if constexpr (PB == 2)
                b1 = __builtin_bit_cast(bf16x8_t,
                                        *(const u32x4_t *)(bw + bplane + qb * 32 * bs + ks * 16));
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const f32x16_t c = (FIRST && ks == 0) ? x16[rb] : acc[qb][rb];
                acc[qb][rb] = mfma32_bf16(ah[rb], b0, c);
                if constexpr (ST == 0) acc[qb][rb] = mfma32_bf16(al[rb], b0, acc[qb][rb]);
                if constexpr (PB == 2) acc[qb][rb] = mfma32_bf16(ah[rb], b1, acc[qb][rb]);
            }
        }
    }
}

// Row norms of the 16 rows lane (l % 32, h = l / 32) holds in a 32-row block
// starting at row r: rows r + 8u + 4h + e in register 4u + e.
__device__ __forceinline__ f32x16_t load_xn16(const float *xn, int64_t r, int h) {
    f32x4_t q[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) q[u] = *(const f32x4_t *)(xn + r + 8 * u + 4 * h);
    return __builtin_bit_cast(f32x16_t, q);
}

template <int ST, int PB, int QB, int RB, int KC, int NW, int MODE>
__global__ __launch_bounds__(64 * NW) void tile_scan_kernel(ScanKArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int NT = 64 * NW;  // threads
    constexpr int BQ = 32 * QB, WR = 32 * RB, BR = NW * WR;
    constexpr int ESZ = ST == 0 ? 4 : 2;
    constexpr int AW = ARows<ST>::W;
    static_assert(KC % 16 == 0, "K-chunk is whole MFMA K-steps");
    static_assert(BR <= kRowSlack, "the last row tile reads at most kRowSlack rows past the end");
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;

    int64_t split, qblk;
    if (!map_block_grouped(a.nqblk, a.nsplit, a.qgroup, &split, &qblk)) return;
    int64_t r0 = split * a.rows_per_split;
    const int64_t r1 = min(a.n, r0 + a.rows_per_split);
    const int64_t q0 = qblk * BQ;
    if (MODE == 1 && a.self_join) r0 = max(r0, q0);  // only ids > query (rows stay 32-aligned)
    if (r0 >= r1) return;

    // LDS: the block's query planes [PB][BQ][ld + 8], then the lists' counters,
    // thresholds and per-wave sort buffers
    uint16_t *qs = (uint16_t *)smem;
    const int kpb = (int)a.ld + 8;
    int *cnt = (int *)(smem + (size_t)PB * BQ * kpb * 2);
    float *thr = (float *)(cnt + NW * BQ);
    float *sv = thr + NW * BQ;
    int *si = (int *)(sv + NW * a.cap);

    for (int t = tid; t < NW * BQ; t += NT) {
        cnt[t] = 0;
        thr[t] = q0 + (t % BQ) < a.nq ? VS_INF : -VS_INF;
    }
    int *cnt_w = cnt + wave * BQ;
    float *thr_w = thr + wave * BQ;
    float *sv_w = sv + wave * a.cap;
    int *si_w = si + wave * a.cap;
    const int64_t list_base = ((qblk * a.nsplit + split) * NW + wave) * (int64_t)BQ * a.cap;
    float *cv = MODE == 0 ? a.cand_v + list_base : nullptr;
    int32_t *ci = MODE == 0 ? a.cand_i + list_base : nullptr;

    const int nkc = (int)(a.ld / KC);
    const int64_t ntiles = (r1 - r0 + BR - 1) / BR;
    const int64_t total = ntiles * nkc;
    const int64_t row_bytes = a.ld * ESZ;
    const char *arow = (const char *)a.xb + (r0 + wave * WR + l32) * row_bytes + 8 * h * ESZ;

    // the block's query planes, whole rows, once
    {
        const int cpr = (int)(a.ld / 8);
        for (int p = tid; p < PB * BQ * cpr; p += NT) {
            const int qr = p / cpr, c = p % cpr;
            *(u32x4_t *)(qs + ((qr % PB) * BQ + qr / PB) * kpb + c * 8) =
                *(const u32x4_t *)(a.qp + ((q0 + qr / PB) * 2 + qr % PB) * a.ld + c * 8);
        }
    }

    float thr_r[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int64_t qg = q0 + qb * 32 + l32;
        if (MODE == 0)
            thr_r[qb] = qg < a.nq ? VS_INF : -VS_INF;
        else
            thr_r[qb] = qg < a.nq ? a.athr[qg] : -VS_INF;
    }

    f32x16_t acc[QB][RB];
    uint32_t gt[QB];
    f32x16_t zero16;
#pragma unroll
    for (int e = 0; e < 16; ++e) zero16[e] = 0.f;
    // x16: the current tile's row norms (the accumulator's start value).  They
    // are read only by a tile's first K-chunk and the next tile's are loaded
    // during its last one; every row has >= 2 K-chunks (ld is a multiple of
    // 2 * KC), so the two never overlap.
    f32x16_t x16[RB];
    u32x4_t abuf[2][KC / 16][RB][AW];

    // prologue: the first chunk's rows and row norms
    a_load<ST, RB, KC>(abuf[0], arow, row_bytes, 0, 0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
        x16[rb] = a.metric == 0 ? load_xn16(a.xn, r0 + wave * WR + rb * 32, h) : zero16;
    __syncthreads();

    int kc = 0;  // current chunk: K-chunk and row tile start
    int64_t t0 = r0;
    // one K-chunk: multiply abuf[CUR] while abuf[CUR ^ 1] receives the next
    // chunk (the loop runs it twice per pass so both indices are constants)
    auto step = [&](auto cur_c, int64_t it) __attribute__((always_inline)) {
        constexpr int CUR = decltype(cur_c)::value, NXT = CUR ^ 1;
        const int64_t wr0 = t0 + wave * WR;  // this wave's first row
        // next chunk: same tile, next K-chunk; or the next tile's first
        const bool more = it + 1 < total;
        const int kc_next = kc + 1 == nkc ? 0 : kc + 1;
        const int64_t t_next = kc + 1 == nkc ? t0 + BR : t0;
        if (kc == 0) {
            if constexpr (MODE == 0) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    gt[qb] = __hip_atomic_load(&a.gthr[q0 + qb * 32 + l32], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (more) {
            a_load<ST, RB, KC>(abuf[NXT], arow, row_bytes, t_next - r0, kc_next);
            if (kc_next == 0 && a.metric == 0) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    x16[rb] = load_xn16(a.xn, t_next + wave * WR + rb * 32, h);
            }
        }
        {
            const uint16_t *bw = qs + l32 * kpb + kc * KC + 8 * h;
            if (kc == 0)
                tile_mma<ST, PB, QB, RB, KC, true>(acc, x16, abuf[CUR], bw, kpb, BQ * kpb);
            else
                tile_mma<ST, PB, QB, RB, KC, false>(acc, x16, abuf[CUR], bw, kpb, BQ * kpb);
        }
        const bool tile_end = kc == nkc - 1;
        kc = kc_next;
        t0 = t_next;
        if (!tile_end) return;
        // ---- epilogue of the tile just finished (this wave: rows wr0 .. wr0 + WR) ----
        // lane (l32, h) holds query l32 of each query block and, in register
        // v of row block rb, row wr0 + 32 rb + 8 (v / 4) + 4 h + v % 4
        if (wr0 + WR > r1) {  // rows past the split end never qualify
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    if (wr0 + rb * 32 + 8 * (v / 4) + 4 * h + v % 4 >= r1) {
#pragma unroll
                        for (int qb = 0; qb < QB; ++qb) acc[qb][rb][v] = VS_INF;
                    }
        }
        if constexpr (MODE == 0) {
            // per query block: one min and one compare per lane decide whether
            // any of its values can enter a list; only blocks with a hit take
            // the append path (rare once the thresholds have converged)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                thr_r[qb] = fminf(thr_r[qb], dec_order(gt[qb]));
                float m = VS_INF;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) m = fminf(m, acc[qb][rb][v]);
                if (!__ballot(m < thr_r[qb])) continue;
                const int q = qb * 32 + l32;
                // make room: a list that this tile could overflow (a query
                // gains at most WR entries per tile and wave) is cut to its
                // kk best first
                if (__ballot(h == 0 && cnt_w[q] > a.cap - WR)) {
                    for (int j = 0; j < 32; ++j) {
                        const int qq = qb * 32 + j;
                        if (cnt_w[qq] > a.cap - WR)
                            flush_list(cv + (int64_t)qq * a.cap, ci + (int64_t)qq * a.cap,
                                       &cnt_w[qq], &thr_w[qq], &thr[qq], BQ, 4, &a.gthr[q0 + qq], sv_w,
                                       si_w, a.cap, a.kk, a.kk_final, a.publish_block, lane);
                    }
                    thr_r[qb] = fminf(thr_r[qb], thr_w[q]);
                }
                // append: one LDS reservation per lane for all its passing values
                int c = 0;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) c += acc[qb][rb][v] < thr_r[qb] ? 1 : 0;
                if (c > 0) {
                    int pos = atomicAdd(&cnt_w[q], c);
                    float *cvq = cv + (int64_t)q * a.cap;
                    int32_t *ciq = ci + (int64_t)q * a.cap;
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const float val = acc[qb][rb][v];
                            if (val < thr_r[qb]) {
                                cvq[pos] = val;
                                ciq[pos] = (int32_t)(wr0 + rb * 32 + 8 * (v / 4) + 4 * h + v % 4);
                                ++pos;
                            }
                        }
                }
                lds_wave_sync();
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
                const int64_t qg = q0 + qb * 32 + l32;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int64_t row = wr0 + rb * 32 + 8 * (v / 4) + 4 * h + v % 4;
                        if (acc[qb][rb][v] <= thr_r[qb] && (!a.self_join || row > qg)) {
                            const unsigned long long pos = atomicAdd(a.count, 1ull);
                            if (pos < (unsigned long long)a.out_cap) {
                                a.out_q[pos] = (int32_t)qg;
                                a.out_i[pos] = (int32_t)row;
                            }
                        }
                    }
                }
            }
        }
    };
    for (int64_t it = 0; it < total; it += 2) {
        step(std::integral_constant<int, 0>{}, it);
        if (it + 1 < total) step(std::integral_constant<int, 1>{}, it + 1);
    }

    if constexpr (MODE == 0) {
        // final: every list holds its kk best in slots [0, kk), padded
        wave_sync();
        for (int q = 0; q < BQ; ++q) {
            const int c = cnt_w[q];
            if (c > a.kk) {
                flush_list(cv + (int64_t)q * a.cap, ci + (int64_t)q * a.cap, &cnt_w[q], &thr_w[q],
                           &thr[q], BQ, 4, &a.gthr[q0 + q], sv_w, si_w, a.cap, a.kk, a.kk_final,
                           a.publish_block, lane);
            } else {
                for (int j = c + lane; j < a.kk; j += 64) {
                    cv[(int64_t)q * a.cap + j] = VS_INF;
                    ci[(int64_t)q * a.cap + j] = -1;
                }
            }
        }
        // a list that cut itself to kk < kk_final entries may have dropped
        // rows at or above its own final threshold: the merge checks that
        // value against the query's final kk_final-th value
        if (a.lbound) {
            wave_sync();
            const int64_t lb = ((qblk * a.nsplit + split) * NW + wave) * (int64_t)BQ;
            for (int q = lane; q < BQ; q += 64) a.lbound[lb + q] = thr_w[q];
        }
    }
}

template <int MODE>
hipError_t launch_tile_scan(int storage, int planes, const ScanPlan &plan, const ScanKArgs &args,
                            hipStream_t st) {
    const int64_t grid = ((tile_grid_space(plan.nqblk, plan.nsplit, plan.tile_group) + 7) / 8) * 8;
    ScanKArgs ga = args;
    ga.qgroup = plan.tile_group;
    void (*fn)(ScanKArgs) = nullptr;
    const int qb = plan.bn / 32;
#define VS_TPICK(ST_, PB_, QB_, RB_, KC_, NW_)                                                \
    if (storage == ST_ && planes == PB_ && qb == QB_ && plan.tile_rb == RB_ &&                  \
        plan.tile_kc == KC_ && plan.lw == NW_)                                                  \
        fn = tile_scan_kernel<ST_, PB_, QB_, RB_, KC_, NW_, MODE>;
    VS_TILE_SHAPES(VS_TPICK)
#undef VS_TPICK
    if (!fn) return hipErrorInvalidValue;
    const size_t lds = plan.lds_bytes;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(64 * plan.lw), lds, st, ga);
    return hipGetLastError();
}

template hipError_t launch_tile_scan<0>(int, int, const ScanPlan &, const ScanKArgs &, hipStream_t);
template hipError_t launch_tile_scan<1>(int, int, const ScanPlan &, const ScanKArgs &, hipStream_t);

}  // namespace vs
