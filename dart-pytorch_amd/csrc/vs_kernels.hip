// vs_kernels.hip -- gfx950 kernels of libvs_hip.so.
//
// Build with -ffp-contract=off: the exact re-rank kernels reproduce the
// reference's separate fp64 multiply and add (index_flat.dart:78-88); a
// fused multiply-add would change the L2 sums.
//
// Data layout in HBM (one index):
//   xb  [cap][ld]  storage rows (fp32 or bf16), row bytes a multiple of 256,
//                  rows past ntotal zero, cap a multiple of 256;
//   xn  [cap]      fp32 of the fp64 sum of squares of each stored row.
// Distance accumulator ("acc space", smaller is better for both metrics):
//   L2: xn[r] - 2 q.x[r]      (the query's own |q|^2 is a per-query constant)
//   IP: -q.x[r]
// The MFMA B operand holds bf16 planes of s*q with s = -2 (L2) or -1 (IP);
// fp32 rows are split in registers into bf16 hi + lo, so an fp32 dot is
// hi*q0 + lo*q0 (+ hi*q1 when the query needs a second plane).
#include <float.h>

#include <algorithm>
#include <limits.h>
#include <math.h>

#include "vs_device.h"

namespace vs {

template <typename T>
__device__ __forceinline__ float load_f32(const T *p, int64_t i);
template <>
__device__ __forceinline__ float load_f32<float>(const float *p, int64_t i) {
    return p[i];
}
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t *p, int64_t i) {
    return bf16_to_f32(p[i]);
}

int64_t storage_ld(int64_t d, int storage) {
    const int64_t es = storage == 1 ? 2 : 4;
    const int64_t bytes = ((d * es + kRowAlignBytes - 1) / kRowAlignBytes) * kRowAlignBytes;
    return bytes / es;
}

// ---------------------------------------------------------------------------
// Row storage: convert / pad / norms / flags.  One wave per row.
// ---------------------------------------------------------------------------
template <typename TS, typename TD>
__global__ __launch_bounds__(256) void store_rows_kernel(const TS *__restrict__ src,
                                                         int64_t src_stride, int64_t n, int64_t d,
                                                         TD *__restrict__ dst, int64_t ld,
                                                         float *__restrict__ xn, uint32_t *flags) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    double ss = 0.0;
    uint32_t f = 0;
    for (int64_t j = lane; j < ld; j += 64) {
        const float v = j < d ? load_f32(src, row * src_stride + j) : 0.0f;
        if (!__builtin_isfinite(v)) f |= kFlagNonFinite;
        const uint16_t h = f32_to_bf16_rne(v);
        if (bf16_to_f32(h) != v) f |= kFlagNotBf16;
        float stored;
        if constexpr (sizeof(TD) == 2) {
            dst[row * ld + j] = h;
            stored = bf16_to_f32(h);
        } else {
            dst[row * ld + j] = v;
            stored = v;
        }
        ss += (double)stored * (double)stored;
    }
    for (int o = 32; o > 0; o >>= 1) {
        ss += __shfl_xor(ss, o);
        f |= __shfl_xor(f, o);
    }
    if (lane == 0) {
        xn[row] = (float)ss;
        // one atomic per new bit: rows of the same data set the same bits, and
        // millions of atomics on one word would serialise
        if (f && (__hip_atomic_load(flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & f) != f)
            atomicOr(flags, f);
    }
}

hipError_t launch_store_rows(const void *src, int src_dtype, int64_t src_stride, int64_t n,
                             int64_t d, void *dst, int dst_dtype, int64_t ld, float *xn,
                             uint32_t *flags, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 3) / 4)), block(256);
    if (src_dtype == 0 && dst_dtype == 0)
        store_rows_kernel<float, float><<<grid, block, 0, st>>>((const float *)src, src_stride, n,
                                                                d, (float *)dst, ld, xn, flags);
    else if (src_dtype == 0 && dst_dtype == 1)
        store_rows_kernel<float, uint16_t><<<grid, block, 0, st>>>(
            (const float *)src, src_stride, n, d, (uint16_t *)dst, ld, xn, flags);
    else if (src_dtype == 1 && dst_dtype == 0)
        store_rows_kernel<uint16_t, float><<<grid, block, 0, st>>>(
            (const uint16_t *)src, src_stride, n, d, (float *)dst, ld, xn, flags);
    else
        store_rows_kernel<uint16_t, uint16_t><<<grid, block, 0, st>>>(
            (const uint16_t *)src, src_stride, n, d, (uint16_t *)dst, ld, xn, flags);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Query preparation.  One wave per (padded) query row.
// ---------------------------------------------------------------------------
template <typename TS>
__global__ __launch_bounds__(256) void prep_queries_kernel(const TS *__restrict__ src,
                                                           int64_t src_stride, int64_t nq,
                                                           int64_t nq_pad, int64_t d, int64_t ld,
                                                           float scale, uint16_t *__restrict__ qp,
                                                           float *__restrict__ qf,
                                                           float *__restrict__ qnorm,
                                                           uint32_t *flags) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= nq_pad) return;
    const bool valid = row < nq;
    double ss = 0.0;
    uint32_t f = 0;
    for (int64_t j = lane; j < ld; j += 64) {
        const bool in = valid && j < d;
        const float v = in ? load_f32(src, row * src_stride + j) : 0.0f;
        if (in) {
            qf[row * d + j] = v;
            if (!__builtin_isfinite(v)) f |= kFlagNonFinite;
        }
        ss += (double)v * (double)v;
        const float s = v * scale;  // scale is -1 or -2: exact
        const uint16_t h0 = f32_to_bf16_rne(s);
        const uint16_t h1 = f32_to_bf16_rne(s - bf16_to_f32(h0));
        if (h1 & 0x7FFFu) f |= kFlagNotBf16;
        qp[(row * 2 + 0) * ld + j] = h0;
        qp[(row * 2 + 1) * ld + j] = h1;
    }
    for (int o = 32; o > 0; o >>= 1) {
        ss += __shfl_xor(ss, o);
        f |= __shfl_xor(f, o);
    }
    if (f & kFlagNonFinite) {
        // the row is prepared as the unit vector e_0 instead: the call reports
        // the flag, and the kernels after this one only ever see finite values
        // (f is the same in every lane)
        for (int64_t j = lane; j < ld; j += 64) {
            if (j < d) qf[row * d + j] = j == 0 ? 1.0f : 0.0f;
            qp[(row * 2 + 0) * ld + j] = j == 0 ? f32_to_bf16_rne(scale) : (uint16_t)0;
            qp[(row * 2 + 1) * ld + j] = 0;
        }
        ss = 1.0;
    }
    if (lane == 0) {
        if (valid) qnorm[row] = (float)sqrt(ss);
        // one atomic per new bit: rows of the same data set the same bits, and
        // millions of atomics on one word would serialise
        if (f && (__hip_atomic_load(flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & f) != f)
            atomicOr(flags, f);
    }
}

hipError_t launch_prepare_queries(const void *src, int src_dtype, int64_t src_stride, int64_t nq,
                                  int64_t d, int64_t ld, int metric, const PreparedQueries &pq,
                                  uint32_t *flags, hipStream_t st) {
    if (pq.nq_pad <= 0) return hipSuccess;
    const float scale = metric == 0 ? -2.0f : -1.0f;
    const dim3 grid((unsigned)((pq.nq_pad + 3) / 4)), block(256);
    if (src_dtype == 0)
        prep_queries_kernel<float><<<grid, block, 0, st>>>((const float *)src, src_stride, nq,
                                                           pq.nq_pad, d, ld, scale, pq.qp, pq.qf,
                                                           pq.qnorm, flags);
    else
        prep_queries_kernel<uint16_t><<<grid, block, 0, st>>>((const uint16_t *)src, src_stride,
                                                              nq, pq.nq_pad, d, ld, scale, pq.qp,
                                                              pq.qf, pq.qnorm, flags);
    return hipGetLastError();
}

// Block-level bitonic sort (blockDim.x threads) of n (power of two) pairs.
__device__ void bitonic_sort_block(float *sv, int *si, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < (n >> 1); t += blockDim.x) {
                const int i = 2 * t - (t & (stride - 1));
                const int j = i + stride;
                const bool asc = (i & size) == 0;
                const float vi = sv[i], vj = sv[j];
                const int ii = si[i], ij = si[j];
                const bool gt = vi > vj || (vi == vj && ii > ij);
                if (gt == asc) {
                    sv[i] = vj;
                    sv[j] = vi;
                    si[i] = ij;
                    si[j] = ii;
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// The fused distance scan.
//
// Grid: one workgroup per (query block, database split), 4 waves.  The
// block's bn queries sit in LDS as bf16 planes; each wave streams its own
// tiles of 16*TM database rows straight from HBM into MFMA A operands
// (16-byte loads; for bf16 rows, 4 lanes x 16 B = 64 contiguous bytes of a
// row per K-step) and multiplies them by all bn queries with
// v_mfma_f32_16x16x32_bf16.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 as used here (lane l, r = l%16,
// g = l/16): A lane holds row r, K elements 8g..8g+7; B lane holds query r,
// the same K elements; D lane holds rows 4g..4g+3 of query r.  A and B use
// the same K assignment, so the dot product does not depend on how the
// hardware orders K inside the instruction.
//
// MODE 0 (top-k): every accumulator below the wave's per-query threshold is
// appended to a per-(wave, query) list in global memory; a list nearing its
// capacity is sorted by the wave and cut to its kk best, which also tightens
// the threshold.  Nothing else of the distance matrix is written.
// MODE 1 (range): accumulators within the per-query bound are appended to a
// global (query, id) candidate list for exact re-testing.
// ---------------------------------------------------------------------------
// planes == 0: the queries live in registers and need no LDS copy.
size_t scan_lds_bytes(int bn, int planes, int64_t ld, int cap, int nw) {
    return (size_t)bn * planes * (size_t)(ld + 8) * 2 + (size_t)nw * bn * 8 + (size_t)nw * cap * 8;
}

typedef float f32x8_t __attribute__((ext_vector_type(8)));
struct U8x2 {
    u32x4_t a, b;
};

template <int ST>
struct AFrag;
template <>
struct AFrag<1> {  // bf16 row: 8 values (16 B) per lane and K-step
    u32x4_t v;
    __device__ __forceinline__ void load(const char *p) { v = *(const u32x4_t *)p; }
};
template <>
struct AFrag<0> {  // fp32 row: 8 values (32 B) per lane and K-step
    U8x2 v;
    __device__ __forceinline__ void load(const char *p) {
        v.a = *(const u32x4_t *)p;
        v.b = *(const u32x4_t *)(p + 16);
    }
};

// NKS > 0: bf16 rows, one query plane, NKS K-steps known at compile time; the
// queries' B fragments stay in registers for the whole kernel and each wave
// prefetches its next tile whole while computing the current one.
// NKS == 0: queries in LDS; rows are consumed in chunks of UK K-steps with the
// next chunk (or the next tile's first chunk) in flight.
template <int ST, int PQ, int NQB, int TM, int MODE, int NKS, int NW>
__global__ __launch_bounds__(64 * NW) void scan_kernel(ScanKArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int BN = 16 * NQB;
    constexpr bool QREG = NKS > 0;
    static_assert(!QREG || (ST == 1 && PQ == 1), "register queries need bf16 rows, one plane");
    constexpr int UK = QREG ? NKS : (ST == 1 ? 4 : 2);
    constexpr int QPL = QREG ? 0 : PQ;  // query planes held in LDS
    constexpr int64_t KSTEP_BYTES = ST == 1 ? 64 : 128;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;

    int64_t split, qblk;
    if (!map_block(a.nqblk, a.nsplit, &split, &qblk)) return;
    int64_t r0 = split * a.rows_per_split;
    const int64_t r1 = min(a.n, r0 + a.rows_per_split);
    if (MODE == 1 && a.self_join) r0 = max(r0, qblk * BN);  // only ids > query
    if (r0 >= r1) return;

    const int64_t ldp = a.ld + 8;
    uint16_t *qs = (uint16_t *)smem;  // [BN][QPL][ldp]
    int *cnt = (int *)(smem + (size_t)BN * QPL * ldp * 2);
    float *thr = (float *)(cnt + NW * BN);
    float *sv = thr + NW * BN;
    int *si = (int *)(sv + NW * a.cap);

    const int64_t q0 = qblk * BN;
    if constexpr (QPL > 0) {
        // the block's query planes into LDS, eight 16-byte loads per thread
        // in flight before their stores (one memory round trip per batch)
        const int cpr = (int)(a.ld / 8);  // 16-byte chunks per plane row
        const int nch = BN * QPL * cpr;
        constexpr int U = 8;
        for (int c0 = threadIdx.x; c0 < nch; c0 += U * 64 * NW) {
            u32x4_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {  // (chunks past the end reload chunk 0)
                const int c = c0 + u * 64 * NW < nch ? c0 + u * 64 * NW : 0;
                const int row = c / cpr, ch = c % cpr;
                const int q = row / QPL, p = row % QPL;
                v[u] = *(const u32x4_t *)(a.qp + ((q0 + q) * 2 + p) * a.ld + ch * 8);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {  // (chunks past the end go to row 0's padding)
                const int c = c0 + u * 64 * NW;
                const bool in = c < nch;
                const int row = in ? c / cpr : 0, ch = in ? c % cpr : cpr;
                *(u32x4_t *)(qs + row * ldp + ch * 8) = v[u];
            }
        }
    }
    for (int t = threadIdx.x; t < NW * BN; t += 64 * NW) {
        cnt[t] = 0;
        thr[t] = q0 + (t % BN) < a.nq ? VS_INF : -VS_INF;
    }
    __syncthreads();

    int *cnt_w = cnt + wave * BN;
    float *thr_w = thr + wave * BN;
    float *sv_w = sv + wave * a.cap;
    int *si_w = si + wave * a.cap;
    const int64_t list_base = ((qblk * a.nsplit + split) * NW + wave) * (int64_t)BN * a.cap;
    float *cv = MODE == 0 ? a.cand_v + list_base : nullptr;
    int32_t *ci = MODE == 0 ? a.cand_i + list_base : nullptr;

    float thr_r[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
        const int64_t qg = q0 + qb * 16 + r16;
        if (MODE == 0)
            thr_r[qb] = thr_w[qb * 16 + r16];
        else
            thr_r[qb] = qg < a.nq ? a.athr[qg] : -VS_INF;
    }

    const int nks = QREG ? NKS : (int)(a.ld / 32);
    const int64_t row_bytes = a.ld * (ST == 1 ? 2 : 4);
    const char *xbase = (const char *)a.xb + (ST == 1 ? g * 16 : g * 32);
    const uint16_t *qlane = qs + (int64_t)r16 * QPL * ldp + 8 * g;

    u32x4_t bq[QREG ? NKS : 1][NQB];
    if constexpr (QREG) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb)
                bq[ks][qb] =
                    *(const u32x4_t *)(a.qp + ((q0 + qb * 16 + r16) * 2) * a.ld + ks * 32 + 8 * g);
    }

    AFrag<ST> cur[UK][TM], nxt[UK][TM];
    f32x4_t xn_cur[TM], xn_nxt[TM];
    const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
        xn_cur[tm] = zero4;
        xn_nxt[tm] = zero4;
    }

    int64_t t0 = r0 + wave * 16 * TM;
    if (t0 < r1) {
#pragma unroll
        for (int u = 0; u < UK; ++u)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                cur[u][tm].load(xbase + (t0 + tm * 16 + r16) * row_bytes + u * KSTEP_BYTES);
        if (a.metric == 0) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                xn_cur[tm] = *(const f32x4_t *)(a.xn + t0 + tm * 16 + 4 * g);
        }
    }

    for (; t0 < r1; t0 += NW * 16 * TM) {
        uint32_t gt[NQB];
        if constexpr (MODE == 0) {
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb)
                gt[qb] = __hip_atomic_load(&a.gthr[q0 + qb * 16 + r16], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        }
        f32x4_t acc[TM][NQB];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) acc[tm][qb] = xn_cur[tm];

        const int64_t tn = t0 + NW * 16 * TM;
        for (int ks = 0; ks < nks; ks += UK) {
            // prefetch: the next chunk of this tile, else the next tile's first
            if (ks + UK < nks) {
#pragma unroll
                for (int u = 0; u < UK; ++u)
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
                        nxt[u][tm].load(xbase + (t0 + tm * 16 + r16) * row_bytes +
                                        (int64_t)(ks + UK + u) * KSTEP_BYTES);
            } else if (tn < r1) {
#pragma unroll
                for (int u = 0; u < UK; ++u)
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
                        nxt[u][tm].load(xbase + (tn + tm * 16 + r16) * row_bytes + u * KSTEP_BYTES);
                if (a.metric == 0) {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
                        xn_nxt[tm] = *(const f32x4_t *)(a.xn + tn + tm * 16 + 4 * g);
                }
            }
#pragma unroll
            for (int u = 0; u < UK; ++u) {
                bf16x8_t hi[TM], lo[TM];
                if constexpr (ST == 0) {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm) {
                        const f32x8_t v = __builtin_bit_cast(f32x8_t, cur[u][tm].v);
                        hi[tm] = __builtin_convertvector(v, bf16x8_t);
                        lo[tm] = __builtin_convertvector(
                            v - __builtin_convertvector(hi[tm], f32x8_t), bf16x8_t);
                    }
                } else {
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm) hi[tm] = __builtin_bit_cast(bf16x8_t, cur[u][tm].v);
                }
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    bf16x8_t b0, b1;
                    if constexpr (QREG) {
                        b0 = __builtin_bit_cast(bf16x8_t, bq[u][qb]);
                    } else {
                        const uint16_t *qrow =
                            qlane + (int64_t)qb * 16 * QPL * ldp + (int64_t)(ks + u) * 32;
                        b0 = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)qrow);
                        if constexpr (PQ == 2)
                            b1 = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(qrow + ldp));
                    }
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm) {
                        acc[tm][qb] = mfma_bf16(hi[tm], b0, acc[tm][qb]);
                        if constexpr (ST == 0) acc[tm][qb] = mfma_bf16(lo[tm], b0, acc[tm][qb]);
                        if constexpr (PQ == 2) acc[tm][qb] = mfma_bf16(hi[tm], b1, acc[tm][qb]);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < UK; ++u)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) cur[u][tm] = nxt[u][tm];
        }
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) xn_cur[tm] = xn_nxt[tm];

        // ---- epilogue ----
        if (t0 + 16 * TM > r1) {  // rows past the split end never qualify
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (t0 + tm * 16 + 4 * g + i >= r1) {
#pragma unroll
                        for (int qb = 0; qb < NQB; ++qb) acc[tm][qb][i] = VS_INF;
                    }
        }
        if constexpr (MODE == 0) {
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) thr_r[qb] = fminf(thr_r[qb], dec_order(gt[qb]));
        }
        // one compare per lane and query block decides whether anything passes
        bool pass = false;
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
            float m = VS_INF;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int i = 0; i < 4; ++i) m = fminf(m, acc[tm][qb][i]);
            pass |= MODE == 0 ? (m < thr_r[qb]) : (m <= thr_r[qb]);
        }
        if (!__ballot(pass)) continue;

        if constexpr (MODE == 0) {
            // make room: a list this tile could overflow (a query gains at
            // most 16 * TM entries per tile) is cut back to its kk best first
            {
                bool need = false;
                if (g == 0) {
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb) need |= cnt_w[qb * 16 + r16] > a.cap - 16 * TM;
                }
                if (__ballot(need)) {
                    for (int q = 0; q < BN; ++q) {
                        if (cnt_w[q] > a.cap - 16 * TM)
                            flush_list(cv + (int64_t)q * a.cap, ci + (int64_t)q * a.cap, &cnt_w[q],
                                       &thr_w[q], &thr[q], BN, 4, &a.gthr[q0 + q], sv_w, si_w, a.cap,
                                       a.kk, a.kk_final, a.publish_block, lane);
                    }
#pragma unroll
                    for (int qb = 0; qb < NQB; ++qb)
                        thr_r[qb] = fminf(thr_r[qb], thr_w[qb * 16 + r16]);
                }
            }
            // append: one LDS reservation per lane and query block for all of
            // the lane's passing values, visiting only blocks with a pass
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
                int c = 0;
#pragma unroll
                for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                    for (int i = 0; i < 4; ++i) c += acc[tm][qb][i] < thr_r[qb] ? 1 : 0;
                if (!__ballot(c > 0)) continue;
                const int q = qb * 16 + r16;
                if (c > 0) {
                    int pos = atomicAdd(&cnt_w[q], c);
                    float *cvq = cv + (int64_t)q * a.cap;
                    int32_t *ciq = ci + (int64_t)q * a.cap;
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float v = acc[tm][qb][i];
                            if (v < thr_r[qb]) {
                                cvq[pos] = v;
                                ciq[pos] = (int32_t)(t0 + tm * 16 + 4 * g + i);
                                ++pos;
                            }
                        }
                }
            }
            lds_wave_sync();
        } else {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int64_t rbase = t0 + tm * 16 + 4 * g;
#pragma unroll
                for (int qb = 0; qb < NQB; ++qb) {
                    const f32x4_t v4 = acc[tm][qb];
                    const float m4 = fminf(fminf(v4[0], v4[1]), fminf(v4[2], v4[3]));
                    if (!__ballot(m4 <= thr_r[qb])) continue;
                    const int64_t qg = q0 + qb * 16 + r16;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int64_t row = rbase + i;
                        if (v4[i] <= thr_r[qb] && (!a.self_join || row > qg)) {
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
    }

    if constexpr (MODE == 0) {
        if (a.list_cnt) {
            // uncut lists: their entry counts (and, after all lists, the
            // largest) for the merge, which filters and selects itself
            wave_sync();
            int32_t *lc = a.list_cnt + ((qblk * a.nsplit + split) * NW + wave) * (int64_t)BN;
            int mx = 0;
            for (int q = lane; q < BN; q += 64) {
                lc[q] = cnt_w[q];
                mx = max(mx, cnt_w[q]);
            }
            for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
            if (lane == 0) atomicMax(a.list_cnt + a.nqblk * a.nsplit * NW * BN, mx);
            return;
        }
        // final: every list holds its kk best in slots [0, kk), padded (one
        // lane per list when the keep fits in registers)
        if (a.kk <= 16) {
            cut_lists_lanes<16>(cv, ci, cnt_w, thr_w, thr, BN, 4, &a.gthr[q0], a.cap, a.kk,
                                a.kk_final, a.publish_block, a.kk, true, lane);
        } else {
            wave_sync();
            for (int q = 0; q < BN; ++q) {
                const int c = cnt_w[q];
                if (c > a.kk) {
                    flush_list(cv + (int64_t)q * a.cap, ci + (int64_t)q * a.cap, &cnt_w[q],
                               &thr_w[q], &thr[q], BN, 4, &a.gthr[q0 + q], sv_w, si_w, a.cap,
                               a.kk, a.kk_final, a.publish_block, lane);
                } else {
                    for (int j = c + lane; j < a.kk; j += 64) {
                        cv[(int64_t)q * a.cap + j] = VS_INF;
                        ci[(int64_t)q * a.cap + j] = -1;
                    }
                }
            }
        }
        // a list that cut itself to kk < kk_final entries may have dropped
        // rows at or above its own final threshold: the merge checks that
        // value against the query's final kk_final-th value
        if (a.lbound) {
            wave_sync();
            const int64_t lb = ((qblk * a.nsplit + split) * NW + wave) * (int64_t)BN;
            for (int q = lane; q < BN; q += 64) a.lbound[lb + q] = thr_w[q];
        }
    }
}

template <int MODE>
static hipError_t launch_scan_mode(int storage, const PreparedQueries &pq, const ScanPlan &plan,
                                   const ScanKArgs &args, hipStream_t st) {
    if (plan.kind == 2) return launch_gemm_scan<MODE>(plan.tile_st, plan.tile_pb, plan, args, st);
    if (plan.kind == 3) return MODE == 0 ? launch_share_scan(plan, args, st) : hipErrorInvalidValue;
    const int64_t total = plan.nqblk * plan.nsplit;
    const int64_t grid = ((total + 7) / 8) * 8;
    const size_t lds = plan.lds_bytes;
    void (*fn)(ScanKArgs) = nullptr;
    const int nqb = plan.bn / 16;
#define VS_PICK(ST_, PQ_, NQB_, TM_, NKS_)                                                  \
    if (storage == ST_ && pq.planes == PQ_ && nqb == NQB_ && plan.tm == TM_ && plan.nks == NKS_ && \
        plan.lw == 4)                                                                              \
        fn = scan_kernel<ST_, PQ_, NQB_, TM_, MODE, NKS_, 4>;
    // eight waves sharing one LDS-resident query block (small batches of long
    // rows, where the block's LDS allows a single workgroup per CU)
#define VS_PICK8(PQ_, NQB_, TM_)                                                             \
    if (storage == 1 && pq.planes == PQ_ && nqb == NQB_ && plan.tm == TM_ && plan.nks == 0 &&   \
        plan.lw == 8)                                                                             \
        fn = scan_kernel<1, PQ_, NQB_, TM_, MODE, 0, 8>;
    VS_PICK8(1, 1, 2) VS_PICK8(1, 2, 2) VS_PICK8(1, 4, 2) VS_PICK8(2, 1, 2) VS_PICK8(2, 2, 2)
    VS_PICK8(2, 4, 2)
#undef VS_PICK8
#define VS_PICK_TM(ST_, PQ_, NQB_, NKS_) \
    VS_PICK(ST_, PQ_, NQB_, 1, NKS_) VS_PICK(ST_, PQ_, NQB_, 2, NKS_) VS_PICK(ST_, PQ_, NQB_, 4, NKS_)
#define VS_PICK_NQB(ST_, PQ_, NKS_) \
    VS_PICK_TM(ST_, PQ_, 1, NKS_) VS_PICK_TM(ST_, PQ_, 2, NKS_) VS_PICK_TM(ST_, PQ_, 4, NKS_)
    VS_PICK_NQB(0, 1, 0)
    VS_PICK_NQB(0, 2, 0)
    VS_PICK_NQB(1, 1, 0)
    VS_PICK_NQB(1, 2, 0)
    VS_PICK_NQB(1, 1, 4)
    VS_PICK_NQB(1, 1, 8)
#undef VS_PICK_NQB
#undef VS_PICK_TM
#undef VS_PICK
    if (!fn) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(64 * plan.lw), lds, st, args);
    return hipGetLastError();
}

hipError_t launch_scan_topk(const void *xb, int storage, int64_t ld, const float *xn, int64_t n,
                            int metric, const PreparedQueries &pq, const ScanPlan &plan,
                            float *cand_v, int32_t *cand_i, uint32_t *gthr, float *lbound,
                            int32_t *list_cnt, hipStream_t st) {
    ScanKArgs a{};
    const bool counted = plan.kind == 3 || (plan.kind == 0 && plan.uncut);
    a.list_cnt = counted ? list_cnt : nullptr;
    if (counted && !list_cnt) return hipErrorInvalidValue;
    a.xb = xb;
    a.ld = ld;
    a.xn = xn;
    a.n = n;
    a.qp = pq.qp;
    a.nq = pq.nq;
    a.nqblk = plan.nqblk;
    a.nsplit = plan.nsplit;
    a.rows_per_split = plan.rows_per_split;
    a.kk = plan.kk;
    a.cap = plan.cap;
    a.metric = metric;
    a.cand_v = cand_v;
    a.cand_i = cand_i;
    a.gthr = gthr;
    a.kk_final = plan.kk_final;
    a.publish_block = 4 * plan.kk >= plan.kk_final;
    a.lbound = plan.kk < plan.kk_final ? lbound : nullptr;
    a.kmin_margin = plan.kmin_margin;
    a.kmin_init = plan.kmin_init;
    a.qorder = plan.qorder;
    a.dev_bound = plan.dev_bound;
    return launch_scan_mode<0>(storage, pq, plan, a, st);
}

hipError_t launch_scan_range(const void *xb, int storage, int64_t ld, const float *xn, int64_t n,
                             const PreparedQueries &pq, const ScanPlan &plan, const float *athr,
                             int self_join, int metric, int32_t *out_q, int32_t *out_i,
                             unsigned long long *count, int64_t cap, hipStream_t st) {
    ScanKArgs a{};
    a.xb = xb;
    a.ld = ld;
    a.xn = xn;
    a.n = n;
    a.qp = pq.qp;
    a.nq = pq.nq;
    a.nqblk = plan.nqblk;
    a.nsplit = plan.nsplit;
    a.rows_per_split = plan.rows_per_split;
    a.kk = plan.kk;
    a.cap = plan.cap;
    a.metric = metric;
    a.kk_final = plan.kk;
    a.athr = athr;
    a.self_join = self_join;
    a.out_q = out_q;
    a.out_i = out_i;
    a.count = count;
    a.out_cap = cap;
    return launch_scan_mode<1>(storage, pq, plan, a, st);
}

// ---------------------------------------------------------------------------
// Merge + exact re-rank.  One workgroup (256 threads) per query.
//   1. stream the query's per-wave lists, keeping entries that beat the
//      current kk-th best, sorting when the LDS buffer fills;
//   2. score the kk survivors exactly in fp64;
//   3. MODE 0: sort by (fp32 score, id), write the k best with sentinels
//      (index.dart:306-313).  MODE 1 (k-means argmin): strict-'<' argmin in
//      id order over the exact scores (kmeans.dart:93-101) plus the proof
//      that no centroid outside the shortlist can beat it.
// ---------------------------------------------------------------------------
struct MergeKArgs {
    const void *xb;
    uint32_t *gthr_w;  // threshold seeding: the shared thresholds to tighten
    int64_t nrows;     // rows of xb: candidate ids must lie in [0, nrows)
    uint32_t *flags;   // kFlagBadId is or-ed in for an id outside them
    const float *pts;  // k-means pick: the points' stored rows (ld values each)
    int64_t ld, d;
    int metric;
    const float *qf;
    int64_t nq;
    int bn, kk, cap;
    int lw;  // lists per (workgroup, query)
    int64_t nsplit;
    const float *cand_v;
    const int32_t *cand_i;
    const uint32_t *gthr;
    int kl;               // entries per list (<= kk)
    const float *lbound;  // per-list own thresholds, or null
    const int32_t *list_cnt;  // per-list entry counts (kl = list capacity), or null; the
                              // largest count follows them, at list_cnt[lists in the scan]
    int64_t nlists_all;       // lists in the scan (index of the largest count)
    // split merge, first pass: part_g workgroups per query, each reducing a
    // slice of the query's list entries to its kk best pairs, written to
    // part_v / part_i [nq][part_g][part_cap] (sentinels +inf, -1); null in
    // every other pass
    int part_g, part_cap;
    float *part_v;
    int32_t *part_i;
    // layout of the lists lbound belongs to (the scan's, also when the
    // lists read are a split merge's partial area)
    int64_t lb_nsplit;
    int lb_lw, lb_bn;
    int32_t *vf_count;    // queries whose lists may have dropped a winner
    int32_t *vf_list;
    int guess;            // thresholds were estimated: flag queries left short
    int seed_rank;        // MODE 2: rank whose value sets the threshold (0: kk)
    float kmin_margin;    // k-means pick over the row-shared scan's k-means lists
    const float *dev_bound;  // k-means pick: the bound on the device (overrides bound; the
                             // margin is then 2.5 times it), or null
    const int32_t *order; // k-means pick: slot s is point order[s] (nq slots), or null:
    int64_t slot0;        // point slot0 + s
    int64_t k;
    float *D;
    int32_t *I;
    // Exactness check of the top-k selection (MODE 0, vx_list non-null).
    // Every row outside the kk kept ones has an accumulator at or above the
    // kk-th kept value, and an accumulator lies within
    //   err(q) = 1.25 (err_r s |q| xmax + err_g (xn_max + s |q| xmax))
    // of the exact xn - 2 q.x (L2, s = 2, xn_max = xmax^2) or -q.x (IP,
    // s = 1, xn_max = 0).  A query whose exact k-th result does not lie
    // below (kk-th kept value - err(q)) is appended to vx_list.
    const float *qnorm;
    float xmax, err_r, err_g;
    int32_t *vx_count;
    int32_t *vx_list;
    // k-means argmin mode
    float bound;
    int32_t *assign;
    double *best_sq;
    int32_t *fb_count;
    int32_t *fb_list;
};

constexpr int kMergeBuf = 2048;
constexpr int kMergeKeepMax = 512;  // kk_final of this build is at most 512

// Block-wide radix selection (256 threads) among the entries t in [0, n)
// that satisfy pred(t): the rank-th smallest key(t) (rank >= 1), found 8
// bits at a time from the top with per-wave histograms in LDS.  Returns the
// key and, in *rank_out, its rank among the entries with exactly that key.
struct SelScratch {
    int hist[4][256];
    int bin, below, eq, n_lt, n_eq, max_id;
};

template <typename KeyF, typename PredF>
__device__ uint32_t radix_select_block(int n, int rank, KeyF key, PredF pred, SelScratch &ss,
                                       int *rank_out, int *eq_out = nullptr) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int t = tid; t < 4 * 256; t += 256) (&ss.hist[0][0])[t] = 0;
        __syncthreads();
        for (int t = tid; t < n; t += 256) {
            if (!pred(t)) continue;
            const uint32_t k = key(t);
            if ((k & mask) == prefix) atomicAdd(&ss.hist[wave][(k >> shift) & 255], 1);
        }
        __syncthreads();
        if (wave == 0) {  // lane owns bins 4 lane .. 4 lane + 3
            int c[4], s = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int b = 4 * lane + u;
                c[u] = ss.hist[0][b] + ss.hist[1][b] + ss.hist[2][b] + ss.hist[3][b];
                s += c[u];
            }
            int inc = s;
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(inc, o);
                if (lane >= o) inc += y;
            }
            int cum = inc - s;
            if (cum < rank && rank <= inc) {  // one lane holds the bin of the rank-th key
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (cum + c[u] >= rank) {
                        ss.bin = 4 * lane + u;
                        ss.below = cum;
                        ss.eq = c[u];  // last round: the entries with exactly the key
                        break;
                    }
                    cum += c[u];
                }
            }
        }
        __syncthreads();
        rank -= ss.below;
        prefix |= (uint32_t)ss.bin << shift;
        mask |= 0xFFu << shift;
    }
    *rank_out = rank;
    if (eq_out) *eq_out = ss.eq;
    return prefix;
}

// The kk smallest (v, id) pairs of sv/si[0, n), n >= kk, in (v, id) order
// -- v finite or +inf, real ids distinct, sentinels (+inf, INT_MAX) --
// move to slots [0, kk) in no particular order; the largest of them is
// returned in (*kth_v, *kth_i).  Selection on the order-preserving code of
// v, then on the ids of the pairs tied at that code.
__device__ void select_block(float *sv, int *si, int n, int kk, float *tmp_v, int *tmp_i,
                             SelScratch &ss, float *kth_v, int *kth_i) {
    const int tid = threadIdx.x;
    int need = 0, unused = 0, eq = 0;
    const uint32_t T = radix_select_block(
        n, kk, [&](int t) { return enc_order(sv[t]); }, [](int) { return true; }, ss, &need, &eq);
    // the pairs tied at the pivot code are all taken when need of them tie
    // (the usual case): the kk-th pair is then the tied one with the largest
    // id, found while they are copied, and the selection on ids is skipped
    const bool all_eq = eq == need;
    const uint32_t I =
        all_eq ? 0xFFFFFFFFu
               : radix_select_block(
                     n, need, [&](int t) { return (uint32_t)si[t]; },
                     [&](int t) { return enc_order(sv[t]) == T; }, ss, &unused);
    // kk - need pairs lie strictly below the pivot code and take slots
    // [0, kk - need); the tied ones take the rest, at most need of them (equal
    // sentinels can tie beyond need)
    if (tid == 0) {
        ss.n_lt = 0;
        ss.n_eq = 0;
        ss.max_id = 0;
    }
    __syncthreads();
    for (int t = tid; t < n; t += 256) {
        const uint32_t c = enc_order(sv[t]);
        int p = -1;
        if (c < T) {
            p = atomicAdd(&ss.n_lt, 1);
        } else if (c == T && (uint32_t)si[t] <= I) {
            const int q = atomicAdd(&ss.n_eq, 1);
            if (q < need) p = kk - need + q;
            if (all_eq) atomicMax(&ss.max_id, si[t]);
        }
        if (p >= 0) {
            tmp_v[p] = sv[t];
            tmp_i[p] = si[t];
        }
    }
    __syncthreads();
    for (int t = tid; t < kk; t += 256) {
        sv[t] = tmp_v[t];
        si[t] = tmp_i[t];
    }
    if (tid == 0) {
        *kth_v = dec_order(T);
        *kth_i = all_eq ? ss.max_id : (int)I;
    }
    __syncthreads();
}

template <int ST, int MODE, int MU>
__global__ __launch_bounds__(256) void merge_refine_kernel(MergeKArgs a) {
    constexpr int MBUF = kMergeBuf * MU;
    extern __shared__ __align__(16) char smem[];
    float *bv = (float *)smem;                  // [MBUF]
    int *bi = (int *)(bv + MBUF);               // [MBUF]
    float *qsh = (float *)(bi + MBUF);          // [ld]
    float *tmp_v = qsh + a.ld;                  // [kMergeKeepMax]
    int *tmp_i = (int *)(tmp_v + kMergeKeepMax);  // [kMergeKeepMax]
    __shared__ SelScratch sel;
    __shared__ int s_cnt;
    __shared__ float s_thr;
    __shared__ int s_thr_id;

    const bool part = a.part_v != nullptr;
    const int64_t qg = part ? blockIdx.x / a.part_g : blockIdx.x;
    const int tid = threadIdx.x;
    const int kk = a.kk;
    // counted lists: only the longest list's fill (rounded up to whole
    // 4-entry reads) needs visiting
    const int kl = a.list_cnt ? max(0, min(a.kl, (a.list_cnt[a.nlists_all] + 3) & ~3)) : a.kl;
    const int64_t qblk = qg / a.bn, q = qg % a.bn;
    const int64_t nlists = a.nsplit * a.lw;
    const int64_t total = nlists * kl;
    // the entries this workgroup visits: all of them, or (split merge) one
    // slice of whole 4-entry groups (kl is a multiple of 4, so a group never
    // straddles two lists)
    int64_t lo = 0, hi = total;
    if (part) {
        const int64_t per = ((total + a.part_g - 1) / a.part_g + 3) & ~(int64_t)3;
        lo = min(total, (int64_t)(blockIdx.x % a.part_g) * per);
        hi = min(total, lo + per);
    }

    for (int t = tid; t < kk; t += 256) {
        bv[t] = VS_INF;
        bi[t] = INT_MAX;
    }
    if (tid == 0) {
        s_cnt = 0;
        s_thr = VS_INF;
        s_thr_id = INT_MAX;
    }
    if (!part)
        for (int64_t j = tid; j < a.ld; j += 256) qsh[j] = j < a.d ? a.qf[qg * a.d + j] : 0.0f;
    __syncthreads();

    // entries above the query's final shared threshold cannot be among the
    // kk best (at least kk candidates lie at or below it); each thread reads
    // 4 adjacent entries of one list per 1024-entry chunk (kl is a multiple
    // of 4), MU chunks per pass with all their loads in flight at once, and
    // the buffer takes a whole pass (MU * 1024 entries) before it is cut
    const float tfinal = a.gthr ? dec_order(a.gthr[qg]) : VS_INF;
    // with several chunks per pass, the first pass takes a single chunk and
    // is cut as soon as it holds 2 kk candidates: its kk-th value then
    // filters the passes after it (lists read without a final threshold would
    // otherwise fill the whole buffer first)
    for (int64_t base = lo; base < hi;) {
        const bool first = base == lo && MU > 1;
        const int nch = first ? 1 : MU;  // chunks of this pass
        float4 v4[MU];
        int4 i4[MU];
        int nv[MU];  // valid entries of the thread's 4 (0 when past the end or the list's count)
#pragma unroll
        for (int u = 0; u < MU; ++u) {
            const int64_t e = base + 1024 * u + 4 * tid;
            nv[u] = 0;
            if (u < nch && e < hi) {
                const int64_t list = e / kl, j = e % kl;
                const int64_t split = list / a.lw, w = list % a.lw;
                const int64_t li = ((qblk * a.nsplit + split) * a.lw + w) * a.bn + q;
                const int64_t lc = a.list_cnt ? a.list_cnt[li] : kl;  // entries past it are stale
                if (j < lc) {
                    const int64_t off = li * a.cap + j;
                    v4[u] = *(const float4 *)(a.cand_v + off);
                    i4[u] = *(const int4 *)(a.cand_i + off);
                    nv[u] = (int)min<int64_t>(4, lc - j);
                }
            }
        }
        const float th = s_thr;
        const int thi = s_thr_id;
#pragma unroll
        for (int u = 0; u < MU; ++u) {
            const float vs4[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
            const int is4[4] = {i4[u].x, i4[u].y, i4[u].z, i4[u].w};
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const float v = vs4[x];
                const int id = is4[x];
                if (x < nv[u] && id >= 0 && v <= tfinal && (v < th || (v == th && id < thi))) {
                    const int pos = atomicAdd(&s_cnt, 1);
                    bv[kk + pos] = v;
                    bi[kk + pos] = id;
                }
            }
        }
        __syncthreads();
        const int c = s_cnt;
        base += 1024 * nch;
        if (c > MBUF - kk - 1024 * MU || (base >= hi && c > 0) || (first && c >= 2 * kk)) {
            // the kk best in any order, and the kk-th
            select_block(bv, bi, kk + c, kk, tmp_v, tmp_i, sel, &s_thr, &s_thr_id);
            if (tid == 0) s_cnt = 0;
        }
        __syncthreads();
    }

    if (part) {
        // the slice's kk best pairs (the kk best of the query are among the
        // union of its slices'), for the second pass
        const int64_t o = (int64_t)blockIdx.x * a.part_cap;
        for (int t = tid; t < a.part_cap; t += 256) {
            const bool ok = t < kk && bi[t] != INT_MAX;
            a.part_v[o + t] = ok ? bv[t] : VS_INF;
            a.part_i[o + t] = ok ? bi[t] : -1;
        }
        return;
    }

    if constexpr (MODE == 2) {
        // threshold seeding: r candidates lie at or below the r-th merged
        // value (r = kk: a bound on the query's kk-th best; r < kk: an
        // estimate of a larger rank of the full scan), and its successor
        // code keeps that value itself below the threshold
        bitonic_sort_block(bv, bi, kk);
        const int r = a.seed_rank > 0 ? a.seed_rank : kk;
        if (tid == 0 && bi[r - 1] != INT_MAX && bv[r - 1] < VS_INF)
            atomicMin(&a.gthr_w[qg], enc_order(bv[r - 1]) + 1u);
        return;
    }

    // Lists that kept only kl < kk entries dropped rows at or above their own
    // final threshold; the merged result is exact when none of those
    // thresholds is below the kk-th kept value.  An estimated threshold
    // dropped every row at or above it; the result is exact when kk
    // candidates were still found below it.  Otherwise flag the query.
    __shared__ int s_vf;  // the query went to vf_list
    if (tid == 0) s_vf = 0;
    if (MODE == 0 && (a.lbound || a.guess)) {
        __shared__ float s_lmin[4];
        float lmin = VS_INF;
        if (a.lbound) {
            const int64_t lq = qg / a.lb_bn, lqq = qg % a.lb_bn;
            for (int64_t l = tid; l < a.lb_nsplit * a.lb_lw; l += 256) {
                const int64_t split = l / a.lb_lw, w = l % a.lb_lw;
                lmin = fminf(lmin,
                             a.lbound[((lq * a.lb_nsplit + split) * a.lb_lw + w) * a.lb_bn + lqq]);
            }
        }
        for (int o = 32; o > 0; o >>= 1) lmin = fminf(lmin, __shfl_xor(lmin, o));
        if ((tid & 63) == 0) s_lmin[tid >> 6] = lmin;
        __syncthreads();
        if (tid == 0) {
            const float m = fminf(fminf(s_lmin[0], s_lmin[1]), fminf(s_lmin[2], s_lmin[3]));
            // (s_thr, s_thr_id): the kk-th kept pair, a sentinel if fewer were found
            const bool short_list = a.guess && s_thr_id == INT_MAX && a.nrows >= kk;
            if (m < s_thr || short_list) {
                a.vf_list[atomicAdd(a.vf_count, 1)] = (int32_t)qg;
                s_vf = 1;
            }
        }
    }

    // exact re-rank of the kk survivors (slots [0, kk), sentinel id INT_MAX);
    // each thread rewrites only its own slots: (key, id) with key = score
    // (L2) or -score (IP), so ascending order is best-first
    double best_ex = __builtin_huge_val();
    int best_id = INT_MAX;
    float a_last = 0.f;
    if constexpr (MODE == 1) a_last = s_thr;
    __syncthreads();
    // When the survivors' rows fit in the buffer past slot kk, the whole
    // workgroup first copies them there, every load in flight at once; each
    // fp64 sum (sequential, in the reference's order) then reads LDS instead
    // of making one HBM round trip per 64 elements.
    const int row_bytes = (int)a.ld * (ST == 1 ? 2 : 4);
    char *stage = (char *)(bv + kk);
    const bool staged = kk * row_bytes <= (MBUF - kk) * 4;
    if (staged) {
        const int ppr = row_bytes / 16, np = kk * ppr;  // 16-byte pieces (ld: 64-element multiple)
        for (int t0 = 0; t0 < np; t0 += 8 * 256) {
            uint4 r[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int t = t0 + u * 256 + tid;
                r[u] = make_uint4(0u, 0u, 0u, 0u);
                if (t < np) {
                    const int id = bi[t / ppr];
                    if (id >= 0 && id != INT_MAX && (int64_t)id < a.nrows)
                        r[u] = *(const uint4 *)((const char *)a.xb + (int64_t)id * row_bytes +
                                                (t % ppr) * 16);
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int t = t0 + u * 256 + tid;
                if (t < np) *(uint4 *)(stage + t * 16) = r[u];
            }
        }
        __syncthreads();
    }
    for (int t = tid; t < kk; t += 256) {
        const int id = bi[t];
        float key = VS_INF;
        if (id != INT_MAX && (id < 0 || (int64_t)id >= a.nrows)) {
            atomicOr(a.flags, kFlagBadId);
            bi[t] = INT_MAX;
        } else if (id != INT_MAX) {
            const double ex = staged ? exact_score<ST>(qsh, stage, a.ld, t, a.d, a.metric)
                                     : exact_score<ST>(qsh, a.xb, a.ld, id, a.d, a.metric);
            key = a.metric == 0 ? (float)ex : -(float)ex;
            if (MODE == 1 && (ex < best_ex || (ex == best_ex && id < best_id))) {
                best_ex = ex;
                best_id = id;
            }
        }
        bv[t] = key;
    }
    __syncthreads();

    if constexpr (MODE == 0) {
        bitonic_sort_block(bv, bi, kk);
        for (int64_t t = tid; t < a.k; t += 256) {
            const bool ok = t < kk && bi[t] != INT_MAX;
            a.D[qg * a.k + t] = ok ? (a.metric == 0 ? bv[t] : -bv[t])
                                   : (a.metric == 0 ? VS_INF : -VS_INF);
            a.I[qg * a.k + t] = ok ? bi[t] : -1;
        }
        // Exactness of the selection: any row outside the kk kept has an
        // exact accumulator >= s_thr - err(q).  The k-th result's exact
        // accumulator (score - |q|^2 for L2, -score for IP; its fp32 key is
        // within 2^-24 relative of the fp64 score) must lie below that, or
        // the query is flagged for the exact path.  Queries already sent to
        // vf_list are searched again anyway.
        if (a.vx_list && tid < 64 && a.k <= kk) {
            double qq = 0.0;
            if (a.metric == 0) {
                for (int64_t j = tid; j < a.d; j += 64) qq += (double)qsh[j] * (double)qsh[j];
                for (int o = 32; o > 0; o >>= 1) qq += __shfl_xor(qq, o);
            }
            if (tid == 0 && !s_vf && bi[a.k - 1] != INT_MAX && s_thr < VS_INF) {
                const double s = a.metric == 0 ? 2.0 : 1.0;
                const double qn = a.qnorm[qg], xm = a.xmax;
                const double err = 1.25 * ((double)a.err_r * s * qn * xm +
                                           (double)a.err_g * ((a.metric == 0 ? xm * xm : 0.0) +
                                                              s * qn * xm)) +
                                   1e-30;
                const double key = bv[a.k - 1];
                double ek = key + fabs(key) * (1.0 / 8388608.0);
                if (a.metric == 0) ek -= qq * (1.0 - 1e-12);  // qq: fp64 sum, error < d 2^-53 qq
                if (!(ek < (double)s_thr - err)) a.vx_list[atomicAdd(a.vx_count, 1)] = (int32_t)qg;
            }
        }
    } else {
        // argmin over (exact score, id): smallest score, lowest id among
        // equals -- the strict '<' scan in centroid order (kmeans.dart:96-101)
        double *dsh = (double *)bv;  // bv is free again: 256 doubles fit
        int *ish = bi;
        __syncthreads();
        dsh[tid] = best_ex;
        ish[tid] = best_id;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if (tid < s) {
                const double v1 = dsh[tid + s];
                const int i1 = ish[tid + s];
                if (v1 < dsh[tid] || (v1 == dsh[tid] && i1 < ish[tid])) {
                    dsh[tid] = v1;
                    ish[tid] = i1;
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            const double best = dsh[0];
            const int bid = ish[0];
            // the shortlist holds the argmin if every centroid outside it is
            // provably worse: its accumulator is >= a_last, and accumulators
            // are within `bound` of xn[c] - 2 x.c = score - |x|^2
            double xx = 0.0;
            for (int64_t j = 0; j < a.d; ++j) xx = xx + (double)qsh[j] * (double)qsh[j];
            const double acc_best = best - xx;
            const bool safe = a_last == VS_INF ||
                              (double)a_last - (double)a.bound > acc_best + 1e-9 * (fabs(xx) + 1.0);
            a.assign[qg] = bid;
            a.best_sq[qg] = best;
            if (!safe) {
                const int pos = atomicAdd(a.fb_count, 1);
                a.fb_list[pos] = (int32_t)qg;
            }
        }
    }
}

static size_t merge_lds(int64_t ld, int mu = 1) {
    return (size_t)kMergeBuf * mu * 8 + (size_t)ld * 4 + (size_t)kMergeKeepMax * 8;
}

size_t merge_lds_bytes(int64_t ld, int mu) { return merge_lds(ld, mu); }

// merge_refine_kernel<ST, MODE, mu> for mu in {1, 2, 4, 8}, or null
template <int ST, int MODE>
static void (*merge_fn(int mu))(MergeKArgs) {
    switch (mu) {
        case 1: return merge_refine_kernel<ST, MODE, 1>;
        case 2: return merge_refine_kernel<ST, MODE, 2>;
        case 4: return merge_refine_kernel<ST, MODE, 4>;
        case 8: return merge_refine_kernel<ST, MODE, 8>;
        default: return nullptr;
    }
}

// One merge pass over the lists, or (plan.merge_g > 1) the split merge's
// two: the first reduces each slice of a query's list entries to its kk best
// pairs, written to the partial area after the lists, and the second merges
// those with the final mode.
static hipError_t launch_merge_passes(void (*fn)(MergeKArgs), size_t lds, MergeKArgs a,
                                      const ScanPlan &plan, int64_t nq, float *cand_v,
                                      int32_t *cand_i, hipStream_t st) {
    if (!fn) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    a.lb_nsplit = plan.nsplit;
    a.lb_lw = plan.lw;
    a.lb_bn = plan.bn;
    const int g = plan.merge_g;
    if (g <= 1) {
        hipLaunchKernelGGL(fn, dim3((unsigned)nq), dim3(256), lds, st, a);
        return hipGetLastError();
    }
    if (plan.kk_final % 4 || nq * g > INT32_MAX) return hipErrorInvalidValue;
    const int64_t off = plan.nqblk * plan.nsplit * plan.lw * plan.bn * plan.cap;
    MergeKArgs a1 = a;
    a1.part_g = g;
    a1.part_cap = plan.kk_final;
    a1.part_v = cand_v + off;
    a1.part_i = cand_i + off;
    hipLaunchKernelGGL(fn, dim3((unsigned)(nq * g)), dim3(256), lds, st, a1);
    if (hipError_t e = hipGetLastError()) return e;
    MergeKArgs a2 = a;
    a2.cand_v = a1.part_v;
    a2.cand_i = a1.part_i;
    a2.list_cnt = nullptr;
    a2.bn = 1;
    a2.lw = 1;
    a2.nsplit = g;
    a2.cap = plan.kk_final;
    a2.kl = plan.kk_final;
    hipLaunchKernelGGL(fn, dim3((unsigned)nq), dim3(256), lds, st, a2);
    return hipGetLastError();
}

hipError_t launch_merge_refine(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                               const PreparedQueries &pq, const ScanPlan &plan,
                               float *cand_v, int32_t *cand_i, const uint32_t *gthr,
                               const float *lbound, int32_t *vf_count, int32_t *vf_list,
                               int64_t k, float *D, int32_t *I, int64_t nrows, uint32_t *flags,
                               int guess, const int32_t *list_cnt, const TopkCheck *chk,
                               hipStream_t st) {
    if (pq.nq <= 0) return hipSuccess;
    MergeKArgs a{};
    a.guess = guess;
    if (chk) {
        a.qnorm = pq.qnorm;
        a.xmax = chk->xmax;
        a.err_r = chk->err_r;
        a.err_g = chk->err_g;
        a.vx_count = chk->vx_count;
        a.vx_list = chk->vx_list;
    }
    const bool counted = plan.kind == 3 || (plan.kind == 0 && plan.uncut);
    a.list_cnt = counted ? list_cnt : nullptr;
    if (counted && !list_cnt) return hipErrorInvalidValue;
    a.xb = xb;
    a.nrows = nrows;
    a.flags = flags;
    a.ld = ld;
    a.d = d;
    a.metric = metric;
    a.qf = pq.qf;
    a.nq = pq.nq;
    a.bn = plan.bn;
    a.lw = plan.lw;
    a.kk = plan.kk_final;
    a.kl = a.list_cnt ? plan.cap : plan.kk;
    a.nlists_all = plan.nqblk * plan.nsplit * plan.lw * plan.bn;

    a.cap = plan.cap;
    a.nsplit = plan.nsplit;
    a.cand_v = cand_v;
    a.cand_i = cand_i;
    a.gthr = gthr;
    a.lbound = plan.kk < plan.kk_final ? lbound : nullptr;
    a.vf_count = vf_count;
    a.vf_list = vf_list;
    a.k = k;
    a.D = D;
    a.I = I;
    void (*fn)(MergeKArgs) =
        storage == 1 ? merge_fn<1, 0>(plan.merge_mu) : merge_fn<0, 0>(plan.merge_mu);
    return launch_merge_passes(fn, merge_lds(ld, plan.merge_mu), a, plan, pq.nq, cand_v, cand_i,
                               st);
}

// ---------------------------------------------------------------------------
// Exact top-kk lists: one workgroup per (query, split) scores every row of
// its split with the reference's fp64 arithmetic (exact_score) and keeps the
// kk best (key, id) pairs, key = fp32 score (L2) or -fp32 score (IP), in
// (key, id) order -- the order the merge's re-rank sorts by.  The lists
// ([nq][nsplit][kk], sentinels (+inf, -1)) then go through the merge, whose
// selection over exact keys is exact.  This is the path for queries whose
// approximate selection could not be proven exact.
// ---------------------------------------------------------------------------
struct ExactKArgs {
    const void *xb;
    int64_t ld, d;
    int metric;
    const float *qf;  // [nq][d]
    int64_t nq, n;
    int kk;
    int64_t nsplit, rows_per_split;
    float *cand_v;
    int32_t *cand_i;
    // row subsets instead of splits (ids non-null): list (q, s) scans the
    // rows ids[seg_off[q nsplit + s] .. + seg_len[q nsplit + s])
    const int32_t *ids;
    const int64_t *seg_off, *seg_len;
    uint32_t *flags;  // kFlagBadId for an id outside [0, n)
};

template <int ST>
__global__ __launch_bounds__(256) void exact_lists_kernel(ExactKArgs a) {
    extern __shared__ __align__(16) char smem[];
    float *bv = (float *)smem;                    // [kMergeBuf]
    int *bi = (int *)(bv + kMergeBuf);            // [kMergeBuf]
    float *qsh = (float *)(bi + kMergeBuf);       // [ld]
    float *tmp_v = qsh + a.ld;                    // [kMergeKeepMax]
    int *tmp_i = (int *)(tmp_v + kMergeKeepMax);  // [kMergeKeepMax]
    __shared__ SelScratch sel;
    __shared__ int s_cnt;
    __shared__ float s_thr;
    __shared__ int s_thr_id;

    const int64_t q = blockIdx.x % a.nq, split = blockIdx.x / a.nq;
    const int tid = threadIdx.x;
    const int kk = a.kk;
    for (int t = tid; t < kk; t += 256) {
        bv[t] = VS_INF;
        bi[t] = INT_MAX;
    }
    if (tid == 0) {
        s_cnt = 0;
        s_thr = VS_INF;
        s_thr_id = INT_MAX;
    }
    for (int64_t j = tid; j < a.ld; j += 256) qsh[j] = j < a.d ? a.qf[q * a.d + j] : 0.0f;
    __syncthreads();
    // rows [r0, r1) of the split, or positions [r0, r1) of the id list
    int64_t r0 = split * a.rows_per_split;
    int64_t r1 = min(a.n, r0 + a.rows_per_split);
    if (a.ids) {
        r0 = a.seg_off[q * a.nsplit + split];
        r1 = r0 + a.seg_len[q * a.nsplit + split];
    }
    for (int64_t base = r0; base < r1; base += 256) {
        const int64_t t = base + tid;
        if (t < r1) {
            int64_t row = t;
            if (a.ids) {
                row = a.ids[t];
                if (row < 0 || row >= a.n) {
                    atomicOr(a.flags, kFlagBadId);
                    row = -1;
                }
            }
            if (row >= 0) {
                const double ex = exact_score<ST>(qsh, a.xb, a.ld, row, a.d, a.metric);
                const float key = a.metric == 0 ? (float)ex : -(float)ex;
                const float th = s_thr;
                const int thi = s_thr_id;
                if (key < th || (key == th && (int)row < thi)) {
                    const int pos = atomicAdd(&s_cnt, 1);
                    bv[kk + pos] = key;
                    bi[kk + pos] = (int)row;
                }
            }
        }
        __syncthreads();
        const int c = s_cnt;
        if (c > kMergeBuf - kk - 256 || (base + 256 >= r1 && c > 0)) {
            select_block(bv, bi, kk + c, kk, tmp_v, tmp_i, sel, &s_thr, &s_thr_id);
            if (tid == 0) s_cnt = 0;
        }
        __syncthreads();
    }
    for (int t = tid; t < kk; t += 256) {
        const int64_t off = (q * a.nsplit + split) * kk + t;
        const bool real = bi[t] != INT_MAX;
        a.cand_v[off] = real ? bv[t] : VS_INF;
        a.cand_i[off] = real ? bi[t] : -1;
    }
}

hipError_t launch_exact_lists(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                              const float *qf, int64_t nq, int64_t n, int kk, int64_t nsplit,
                              int64_t rows_per_split, float *cand_v, int32_t *cand_i,
                              hipStream_t st, const int32_t *ids, const int64_t *seg_off,
                              const int64_t *seg_len, uint32_t *flags) {
    if (nq <= 0) return hipSuccess;
    if (kk < 4 || kk > kMergeKeepMax || (kk & 3) || nsplit < 1 || nq * nsplit > INT32_MAX)
        return hipErrorInvalidValue;
    if (ids && (!seg_off || !seg_len || !flags)) return hipErrorInvalidValue;
    ExactKArgs a{xb,     ld,     d,      metric,         qf,      nq,      n,
                 kk,     nsplit, rows_per_split, cand_v, cand_i, ids, seg_off,
                 seg_len, flags};
    const size_t lds = merge_lds(ld);
    void (*fn)(ExactKArgs) = storage == 1 ? exact_lists_kernel<1> : exact_lists_kernel<0>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)(nq * nsplit)), dim3(256), lds, st, a);
    return hipGetLastError();
}

// out[r] = fp32 of the exact fp64 score of row r against one query
template <int ST>
__global__ __launch_bounds__(256) void exact_all_kernel(const void *xb, int64_t ld, int64_t d,
                                                        int metric, const float *qf, int64_t n,
                                                        float *out) {
    extern __shared__ __align__(16) char smem[];
    float *qsh = (float *)smem;  // [ld], zero past d
    for (int64_t j = threadIdx.x; j < ld; j += 256) qsh[j] = j < d ? qf[j] : 0.0f;
    __syncthreads();
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n) out[r] = (float)exact_score<ST>(qsh, xb, ld, r, d, metric);
}

hipError_t launch_exact_all(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                            const float *qf, int64_t n, float *out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const size_t lds = (size_t)ld * 4;
    void (*fn)(const void *, int64_t, int64_t, int, const float *, int64_t, float *) =
        storage == 1 ? exact_all_kernel<1> : exact_all_kernel<0>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)((n + 255) / 256)), dim3(256), lds, st, xb, ld, d, metric,
                       qf, n, out);
    return hipGetLastError();
}

// dst[i][0..w) = src[list[i]][0..w), 32-bit words
__global__ void gather_rows_kernel(const uint32_t *__restrict__ src, const int32_t *__restrict__ list,
                                   int64_t m, int64_t w, uint32_t *__restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= m * w) return;
    const int64_t i = t / w, j = t % w;
    dst[t] = src[(int64_t)list[i] * w + j];
}

// dst[list[i]][0..w) = src[i][0..w), 32-bit words
__global__ void scatter_rows_kernel(const uint32_t *__restrict__ src, const int32_t *__restrict__ list,
                                    int64_t m, int64_t w, uint32_t *__restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= m * w) return;
    const int64_t i = t / w, j = t % w;
    dst[(int64_t)list[i] * w + j] = src[t];
}

hipError_t launch_gather_rows(const void *src, const int32_t *list, int64_t m, int64_t w,
                              void *dst, hipStream_t st) {
    if (m <= 0 || w <= 0) return hipSuccess;
    gather_rows_kernel<<<dim3((unsigned)((m * w + 255) / 256)), dim3(256), 0, st>>>(
        (const uint32_t *)src, list, m, w, (uint32_t *)dst);
    return hipGetLastError();
}

hipError_t launch_scatter_rows(const void *src, const int32_t *list, int64_t m, int64_t w,
                               void *dst, hipStream_t st) {
    if (m <= 0 || w <= 0) return hipSuccess;
    scatter_rows_kernel<<<dim3((unsigned)((m * w + 255) / 256)), dim3(256), 0, st>>>(
        (const uint32_t *)src, list, m, w, (uint32_t *)dst);
    return hipGetLastError();
}

// fill n 32-bit words with v (a kernel rather than a memset node)
__global__ void fill32_kernel(uint32_t *p, int64_t n, uint32_t v) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n) p[t] = v;
}

hipError_t launch_fill32(void *p, int64_t n, uint32_t v, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    fill32_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>((uint32_t *)p, n, v);
    return hipGetLastError();
}

template <int KK>
__global__ void kmeans_pick_kernel(MergeKArgs a);
// The two LDS-staged picks get the register budget of the occupancy their
// LDS allows (two workgroups per CU with 16-dimension chunks, three with 8);
// the compiler's default budget, four waves, spilled the candidates' fp64
// sums.  (The attribute takes effect on this first declaration.)
template <int E, int CH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void
kmeans_pick_wave_kernel(MergeKArgs a);
template <int E, int CH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 3))) void
kmeans_pick_set_kernel(MergeKArgs a);
constexpr int kPickSetMaxK = 16384;  // the distinct-candidate pick's largest K

// Threshold estimates from a pre-pass (seed_rank <= 64): one wave per query.
// Every lane keeps the 8 smallest values it reads from the query's lists,
// sorted in registers; then seed_rank rounds of a wave-wide minimum pop the
// smallest remaining value (from the lowest lane holding it).  The last one
// popped is the seed_rank-th smallest of the lists whenever no lane held
// more than 8 of those, and larger otherwise (never smaller, so the rows of
// the sample at or below it are at least seed_rank).  With fewer than
// seed_rank values the threshold stays.
__global__ __launch_bounds__(256) void merge_estimate_kernel(MergeKArgs a) {
    constexpr int L = 8;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t qg = (int64_t)blockIdx.x * 4 + wave;
    if (qg >= a.nq) return;
    const int64_t qblk = qg / a.bn, q = qg % a.bn;
    const int64_t nlists = a.nsplit * a.lw;
    const float tfinal = dec_order(a.gthr[qg]);
    float loc[L];
#pragma unroll
    for (int i = 0; i < L; ++i) loc[i] = VS_INF;
    for (int64_t l = 0; l < nlists; ++l) {
        const int64_t split = l / a.lw, w = l % a.lw;
        const int64_t li = ((qblk * a.nsplit + split) * a.lw + w) * a.bn + q;
        const int64_t lc = a.list_cnt ? min((int64_t)a.kl, (int64_t)a.list_cnt[li]) : a.kl;
        for (int64_t e = lane; e < lc; e += 64) {
            float v = a.cand_v[li * a.cap + e];
            if (a.cand_i[li * a.cap + e] < 0 || !(v <= tfinal) || !(v < loc[L - 1])) continue;
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const float lo = fminf(loc[i], v);
                v = fmaxf(loc[i], v);
                loc[i] = lo;
            }
        }
    }
    float kth = VS_INF;
    for (int k = 0; k < a.seed_rank; ++k) {
        float m = loc[0];
        for (int o = 32; o > 0; o >>= 1) m = fminf(m, __shfl_xor(m, o));
        if (!(m < VS_INF)) break;  // fewer than seed_rank values
        const unsigned long long holders = __ballot(loc[0] == m);
        if (lane == __ffsll((long long)holders) - 1) {
#pragma unroll
            for (int i = 0; i + 1 < L; ++i) loc[i] = loc[i + 1];
            loc[L - 1] = VS_INF;
        }
        if (k + 1 == a.seed_rank) kth = m;
    }
    if (lane == 0 && kth < VS_INF) atomicMin(&a.gthr_w[qg], enc_order(kth) + 1u);
}

// Threshold seeding from a pre-pass: for every query, the kk_final-th
// smallest accumulator value over its lists tightens its shared threshold.
hipError_t launch_merge_threshold(const PreparedQueries &pq, const ScanPlan &plan,
                                  float *cand_v, int32_t *cand_i, uint32_t *gthr,
                                  int64_t ld, int seed_rank, const int32_t *list_cnt,
                                  hipStream_t st) {
    if (pq.nq <= 0) return hipSuccess;
    if (seed_rank < 0 || seed_rank > plan.kk_final) return hipErrorInvalidValue;
    MergeKArgs a{};
    a.seed_rank = seed_rank;
    const bool counted = plan.kind == 3 || (plan.kind == 0 && plan.uncut);
    a.list_cnt = counted ? list_cnt : nullptr;
    if (counted && !list_cnt) return hipErrorInvalidValue;
    a.ld = ld;
    a.d = 0;
    a.qf = pq.qf;
    a.nq = pq.nq;
    a.bn = plan.bn;
    a.lw = plan.lw;
    a.kk = plan.kk_final;
    a.kl = a.list_cnt ? plan.cap : plan.kk;
    a.nlists_all = plan.nqblk * plan.nsplit * plan.lw * plan.bn;  // the largest count's slot
    a.cap = plan.cap;
    a.nsplit = plan.nsplit;
    a.cand_v = cand_v;
    a.cand_i = cand_i;
    a.gthr = gthr;
    a.gthr_w = gthr;
    if (seed_rank > 0 && seed_rank <= 64) {
        merge_estimate_kernel<<<dim3((unsigned)((pq.nq + 3) / 4)), dim3(256), 0, st>>>(a);
        return hipGetLastError();
    }
    return launch_merge_passes(merge_fn<1, 2>(plan.merge_mu), merge_lds(ld, plan.merge_mu), a,
                               plan, pq.nq, cand_v, cand_i, st);
}

hipError_t launch_kmeans_pick(const float *x, int64_t ld, int64_t d, int64_t n, const float *cen,
                              int64_t K, const float *cand_v, const int32_t *cand_i,
                              const uint32_t *gthr, const ScanPlan &plan, float bound,
                              const float *qf, int32_t *assign,
                              double *best_sq, int32_t *fallback_count, int32_t *fallback_list,
                              uint32_t *flags, const int32_t *list_cnt, const int32_t *order,
                              hipStream_t st, int64_t slot0, int64_t nslots) {
    if (n <= 0) return hipSuccess;
    if (nslots < 0) nslots = n;
    if (slot0 < 0 || slot0 + nslots > n ||
        ((slot0 > 0 || nslots < n) && !(plan.kind == 3 && plan.share_kmin)))
        return hipErrorInvalidValue;
    if (nslots == 0) return hipSuccess;
    MergeKArgs a{};
    a.xb = cen;
    a.pts = x;
    a.nrows = K;
    a.flags = flags;
    a.ld = ld;
    a.d = d;
    a.metric = 0;
    a.qf = qf;
    a.nq = n;
    a.bn = plan.bn;
    a.lw = plan.lw;
    a.kk = plan.kk_final;
    a.kl = plan.kk;
    a.cap = plan.cap;
    a.nsplit = plan.nsplit;
    a.cand_v = cand_v;
    a.cand_i = cand_i;
    a.gthr = gthr;
    a.bound = bound;
    a.dev_bound = plan.dev_bound;
    a.assign = assign;
    a.best_sq = best_sq;
    a.fb_count = fallback_count;
    a.fb_list = fallback_list;
    if (plan.kind == 3 && plan.share_kmin) {
        // count-terminated k-means lists of the row-shared scan
        if (!list_cnt || ld % 16 || plan.share_topm ||
            !(plan.kmin_margin > 0.f || plan.dev_bound))
            return hipErrorInvalidValue;
        a.list_cnt = list_cnt;
        a.kmin_margin = plan.kmin_margin;
        a.kl = plan.cap;
        a.order = order;
        a.slot0 = slot0;
        a.nq = nslots;
        // points grouped by the previous step's clusters share candidates:
        // each distinct one is staged once per wave; in index order (the
        // first step) they share few, and slot-by-slot staging is faster
        // (measured on C4: 1.99 against 2.70 ms grouped, 5.61 against
        // 4.19 ms in index order).  8-dimension chunks leave LDS for three
        // workgroups per CU (C4 pick 1.72 -> 1.56 ms against 16)
        if (K <= kPickSetMaxK && order)
            kmeans_pick_set_kernel<32, 8>
                <<<dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, st>>>(a);
        else
            kmeans_pick_wave_kernel<32, 16>
                <<<dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, st>>>(a);
        return hipGetLastError();
    }
    if (plan.kind == 3) return hipErrorInvalidValue;  // row-shared lists are k-means lists only
    if (plan.kk_final == 16 && plan.kk == 16) {
        kmeans_pick_kernel<16><<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(a);
        return hipGetLastError();
    }
    const size_t lds = merge_lds(ld);
    void (*fn)(MergeKArgs) = merge_refine_kernel<0, 1, 1>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)fn,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)n), dim3(256), lds, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k-means shortlist pick, one lane per point (the lists of a point hold at
// most KK candidates each, KK = the shortlist length kk_final).  The lane
// keeps the KK smallest (accumulator, id) pairs of its lists in registers,
// re-scores exactly -- fp64, dimensions in order, as kmeans.dart:93-101 --
// only the candidates whose accumulator lies within 2 * bound of the best
// one (any other is provably worse than that one), and takes the argmin
// with the lowest id among equal scores.  The pick is proven when every
// centroid outside the shortlist (accumulator >= the KK-th smallest a_last)
// is provably worse; unproven points go to the exhaustive kernel.
// ---------------------------------------------------------------------------
template <int KK>
__global__ __launch_bounds__(256) void kmeans_pick_kernel(MergeKArgs a) {
    if (a.dev_bound) a.bound = *a.dev_bound;
    const int64_t qg = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (qg >= a.nq) return;
    const int64_t qblk = qg / a.bn, q = qg % a.bn;
    float bv[KK];
    int bi[KK];
#pragma unroll
    for (int i = 0; i < KK; ++i) {
        bv[i] = VS_INF;
        bi[i] = INT_MAX;
    }
    // entries above the point's final shared threshold are not among the KK
    // smallest (at least KK candidates lie at or below it)
    const float tfinal = a.gthr ? dec_order(a.gthr[qg]) : VS_INF;
    const int64_t nlists = a.nsplit * a.lw;
    for (int64_t l = 0; l < nlists; ++l) {
        const int64_t split = l / a.lw, w = l % a.lw;
        const int64_t off = (((qblk * a.nsplit + split) * a.lw + w) * a.bn + q) * a.cap;
        for (int j = 0; j < a.kl; j += 4) {  // kl is a multiple of 4
            const float4 v4 = *(const float4 *)(a.cand_v + off + j);
            const int4 i4 = *(const int4 *)(a.cand_i + off + j);
            const float vs4[4] = {v4.x, v4.y, v4.z, v4.w};
            const int is4[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float cv = vs4[u];
                int ci = is4[u];
                if (ci < 0 || cv > tfinal) continue;
                if (!(cv < bv[KK - 1] || (cv == bv[KK - 1] && ci < bi[KK - 1]))) continue;
#pragma unroll
                for (int i = 0; i < KK; ++i) {  // insertion into the sorted pairs
                    const bool lt = cv < bv[i] || (cv == bv[i] && ci < bi[i]);
                    const float tv = lt ? bv[i] : cv;
                    const int ti = lt ? bi[i] : ci;
                    bv[i] = lt ? cv : bv[i];
                    bi[i] = lt ? ci : bi[i];
                    cv = tv;
                    ci = ti;
                }
            }
        }
    }
    // exact scores: the point's stored row and the centroid rows, both ld
    // values with zeros past d (the padding adds +0.0), read 16 bytes at a
    // time and summed in dimension order; |x|^2 in order alongside the first
    const float4 *xr = (const float4 *)(a.pts + qg * a.ld);
    const float *cen = (const float *)a.xb;
    const float lim = bv[0] + 2.0f * a.bound;
    const int64_t n4 = a.ld / 4;
    double best = __builtin_huge_val(), xx = 0.0;
    int bid = INT_MAX;
#pragma unroll
    for (int i = 0; i < KK; ++i) {
        if (bi[i] != INT_MAX && (bi[i] < 0 || (int64_t)bi[i] >= a.nrows)) {
            atomicOr(a.flags, kFlagBadId);
        } else if (bi[i] != INT_MAX && (i == 0 || bv[i] <= lim)) {
            const float4 *cr = (const float4 *)(cen + (int64_t)bi[i] * a.ld);
            double s = 0.0;
            for (int64_t j4 = 0; j4 < n4; ++j4) {
                const float4 xv = xr[j4];
                const float4 cv = cr[j4];
                const double d0 = (double)xv.x - (double)cv.x, d1 = (double)xv.y - (double)cv.y;
                const double d2 = (double)xv.z - (double)cv.z, d3 = (double)xv.w - (double)cv.w;
                s = s + d0 * d0;
                s = s + d1 * d1;
                s = s + d2 * d2;
                s = s + d3 * d3;
                if (i == 0) {
                    xx = xx + (double)xv.x * (double)xv.x;
                    xx = xx + (double)xv.y * (double)xv.y;
                    xx = xx + (double)xv.z * (double)xv.z;
                    xx = xx + (double)xv.w * (double)xv.w;
                }
            }
            if (s < best || (s == best && bi[i] < bid)) {
                best = s;
                bid = bi[i];
            }
        }
    }
    // accumulators are within `bound` of |c|^2 - 2 x.c = score - |x|^2
    const float a_last = bv[KK - 1];
    const bool safe = bid != INT_MAX &&
                      (a_last == VS_INF ||
                       (double)a_last - (double)a.bound > (best - xx) + 1e-9 * (fabs(xx) + 1.0));
    a.assign[qg] = bid == INT_MAX ? 0 : bid;
    a.best_sq[qg] = best;
    if (!safe) a.fb_list[atomicAdd(a.fb_count, 1)] = (int32_t)qg;
}

// The pick's first phase for one point (row qc of the scan's query blocks):
// vmin, the smallest value of its count-terminated k-means lists, the bound
// vmin + kmin_margin that every centroid outside them reaches, and its
// candidates -- the ids within 2 * bound of vmin -- handed to put(slot, id)
// in list order.  Returns their number; *over is set when a list was marked
// full or more than E candidates were found (the point then goes to the
// exhaustive kernel).
template <int E, typename Put>
__device__ __forceinline__ int pick_candidates(const MergeKArgs &a, int64_t qc, float *vmin_out,
                                               float *seg_bound_out, bool *over_io, Put put) {
    const int64_t qblk = qc / a.bn, q = qc % a.bn;
    const int64_t nlists = a.nsplit * a.lw;
    auto list_off = [&](int64_t l) {
        const int64_t split = l / a.lw, w = l % a.lw;
        return (((qblk * a.nsplit + split) * a.lw + w) * a.bn + q) * a.cap;
    };
    float vmin = VS_INF;
    bool over = *over_io;
    auto list_len = [&](int64_t l) -> int {
        const int64_t split = l / a.lw, w = l % a.lw;
        const int c = a.list_cnt[((qblk * a.nsplit + split) * a.lw + w) * a.bn + q];
        return c > a.cap ? 0 : c;
    };
    // 16 entries (four 16-byte reads, all in flight) per step: a list's
    // capacity is a power of two >= 16, so a step never leaves its buffer;
    // entries past the count are skipped by index
    constexpr int G = 16;
    for (int64_t l = 0; l < nlists; ++l) {
        const int64_t off = list_off(l);
        const int64_t split = l / a.lw, w = l % a.lw;
        if (a.list_cnt[((qblk * a.nsplit + split) * a.lw + w) * a.bn + q] > a.cap) over = true;
        // every appended entry has a real id
        const int lc = list_len(l);
        for (int e0 = 0; e0 < lc; e0 += G) {
            float4 v4[G / 4];
#pragma unroll
            for (int u = 0; u < G / 4; ++u) v4[u] = *(const float4 *)(a.cand_v + off + e0 + 4 * u);
#pragma unroll
            for (int u = 0; u < G / 4; ++u) {
                const float v[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (e0 + 4 * u + k < lc) vmin = fminf(vmin, v[k]);
            }
        }
    }
    // every centroid outside the lists: accumulator >= vmin + margin (the
    // scan's fp32 sum, monotone in vmin)
    const float lim = vmin + 2.0f * a.bound;
    int ne = 0;
    for (int64_t l = 0; l < nlists; ++l) {
        const int64_t off = list_off(l);
        const int lc = list_len(l);
        for (int e0 = 0; e0 < lc; e0 += G) {
            float4 v4[G / 4];
            int4 i4[G / 4];
#pragma unroll
            for (int u = 0; u < G / 4; ++u) {
                v4[u] = *(const float4 *)(a.cand_v + off + e0 + 4 * u);
                i4[u] = *(const int4 *)(a.cand_i + off + e0 + 4 * u);
            }
#pragma unroll
            for (int u = 0; u < G / 4; ++u) {
                const float v[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
                const int ids[4] = {i4[u].x, i4[u].y, i4[u].z, i4[u].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (e0 + 4 * u + k >= lc || v[k] > lim) continue;
                    const int id = ids[k];
                    if (id < 0) continue;
                    if ((int64_t)id >= a.nrows) {
                        atomicOr(a.flags, kFlagBadId);
                        continue;
                    }
                    if (ne < E)
                        put(ne++, id);
                    else
                        over = true;
                }
            }
        }
    }
    *vmin_out = vmin;
    *seg_bound_out = vmin + a.kmin_margin;
    *over_io = over;
    return ne;
}

// ---------------------------------------------------------------------------
// k-means pick over the row-shared scan's k-means lists, the exact
// re-scoring staged through LDS: one wave per 64 points (lane = point).  Each lane gathers the ids of its candidates
// within 2 * bound of its smallest accumulator (at most E; a point with more
// goes to the exhaustive kernel, whose exact argmin is the same answer).
// The rows are then walked in chunks of CH dimensions: the chunk of the
// wave's 64 points, and for every candidate slot the chunk of the 64 lanes'
// candidate centroids, are read with 16-byte loads (four lanes per 64-byte
// row piece) into LDS laid out dimension-major, and every lane continues its
// own fp64 sums in dimension order -- the order, and so the rounding, of
// the one-lane-per-point kernel above.
//
// The lists are count-terminated: every scan lane appended what lay below
// its running minimum + kmin_margin, so every centroid outside the lists has
// an accumulator at or above vmin + kmin_margin, rounded as the scan rounds
// it; a list marked full, count cap + 1, sends its point to the exhaustive
// kernel.
// ---------------------------------------------------------------------------
template <int E, int CH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void kmeans_pick_wave_kernel(
    MergeKArgs a) {
    if (a.dev_bound) {
        a.bound = *a.dev_bound;
        a.kmin_margin = 2.5f * a.bound;
    }
    constexpr int RS = 65;  // LDS words per staged dimension (64 rows + 1: no bank conflicts on reads)
    constexpr int PIECES = CH / 4;            // 16-byte pieces per row chunk
    constexpr int ROWS_PER = 64 / PIECES;     // rows covered by one wave-wide load
    static_assert(CH % 4 == 0 && 64 % PIECES == 0, "whole 16-byte pieces");
    __shared__ float xs_all[4][CH * RS];
    __shared__ float cs_all[4][CH * RS];
    __shared__ int id_all[4][E * 64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *xs = xs_all[wave], *cs = cs_all[wave];
    int *ids = id_all[wave];
    const int64_t p0 = ((int64_t)blockIdx.x * 4 + wave) * 64;
    if (p0 >= a.nq) return;  // whole waves only: every lane below stays to the end
    // slot s of the walk is point order[s] (the previous step's grouping by
    // cluster: a wave's points then share most candidates), or slot0 + s
    auto point = [&](int64_t s) -> int64_t { return a.order ? (int64_t)a.order[s] : a.slot0 + s; };
    const bool live = p0 + lane < a.nq;
    // lanes past the end mirror the wave's first point
    const int64_t qg = point(live ? p0 + lane : p0);
    const int64_t qc = qg;
    float vmin = VS_INF, seg_bound = VS_INF;
    bool over = false;
    const int ne = pick_candidates<E>(a, qc, &vmin, &seg_bound, &over,
                                      [&](int e, int id) { ids[e * 64 + lane] = id; });
    int emax = live && !over ? ne : 0;
    for (int o = 32; o > 0; o >>= 1) emax = max(emax, __shfl_xor(emax, o));
    for (int e = ne; e < emax; ++e) ids[e * 64 + lane] = -1;
    lds_wave_sync();

    const int prow = lane / PIECES, pcol = (lane % PIECES) * 4;  // this lane's load piece
    double sc[E], xx = 0.0;
#pragma unroll
    for (int e = 0; e < E; ++e) sc[e] = 0.0;
    for (int64_t c0 = 0; c0 < a.ld; c0 += CH) {
        // the chunk of the wave's points (rows past the end read the first)
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int r = i * ROWS_PER + prow;
            const int64_t pr = point(p0 + r < a.nq ? p0 + r : p0);
            const float4 v = *(const float4 *)(a.pts + pr * a.ld + c0 + pcol);
            xs[(pcol + 0) * RS + r] = v.x;
            xs[(pcol + 1) * RS + r] = v.y;
            xs[(pcol + 2) * RS + r] = v.z;
            xs[(pcol + 3) * RS + r] = v.w;
        }
        lds_wave_sync();
        float xr[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            xr[j] = xs[j * RS + lane];
            xx = xx + (double)xr[j] * (double)xr[j];
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if (e < emax) {  // uniform: every slot index stays a constant
                lds_wave_sync();  // the previous slot's reads of cs are done
#pragma unroll
                for (int i = 0; i < PIECES; ++i) {
                    const int r = i * ROWS_PER + prow;
                    const int id = ids[e * 64 + r];
                    const float4 v = *(const float4 *)((const float *)a.xb +
                                                       (int64_t)(id >= 0 ? id : 0) * a.ld + c0 + pcol);
                    cs[(pcol + 0) * RS + r] = v.x;
                    cs[(pcol + 1) * RS + r] = v.y;
                    cs[(pcol + 2) * RS + r] = v.z;
                    cs[(pcol + 3) * RS + r] = v.w;
                }
                lds_wave_sync();
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    const double dd = (double)xr[j] - (double)cs[j * RS + lane];
                    sc[e] = sc[e] + dd * dd;
                }
            }
        }
        lds_wave_sync();  // xs and cs are rewritten by the next chunk
    }
    if (!live) return;
    double best = __builtin_huge_val();
    int bid = INT_MAX;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int id = e < ne ? ids[e * 64 + lane] : INT_MAX;
        if (e < ne && (sc[e] < best || (sc[e] == best && id < bid))) {
            best = sc[e];
            bid = id;
        }
    }
    const bool safe = !over && bid != INT_MAX &&
                      (seg_bound == VS_INF ||
                       (double)seg_bound - (double)a.bound > (best - xx) + 1e-9 * (fabs(xx) + 1.0));
    a.assign[qg] = bid == INT_MAX ? 0 : bid;
    a.best_sq[qg] = best;
    if (!safe) a.fb_list[atomicAdd(a.fb_count, 1)] = (int32_t)qg;
}

// ---------------------------------------------------------------------------
// The same pick with each distinct candidate centroid read once per wave.
// The wave's points walk in cluster order, so its 64 lanes share most of
// their candidates: the union of their ids (a bitmap over the K <=
// kPickSetMaxK centroids, ranked by a prefix count over its words) numbers
// the distinct centroids 0 .. u - 1, and every lane's candidate becomes a
// slot in that numbering.  Each CH-dimension chunk then stages the points'
// chunk and the distinct centroids' chunks (64 slots per batch, usually one
// batch) with all loads in flight at once, and every lane continues its
// candidates' fp64 sums in dimension order, as the kernel above does (same
// order, same rounding), reading the centroid values by slot.  A wave whose
// union exceeds kPickSetMaxU sends its points to the exhaustive kernel.
// ---------------------------------------------------------------------------
constexpr int kPickSetMaxU = 1024;

template <int E, int CH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 3))) void kmeans_pick_set_kernel(
    MergeKArgs a) {
    if (a.dev_bound) {
        a.bound = *a.dev_bound;
        a.kmin_margin = 2.5f * a.bound;
    }
    constexpr int RS = 65;  // LDS words per staged dimension (64 rows + 1: no bank conflicts on reads)
    constexpr int PIECES = CH / 4;            // 16-byte pieces per row chunk
    constexpr int ROWS_PER = 64 / PIECES;     // rows covered by one wave-wide load
    constexpr int KW = kPickSetMaxK / 64;     // bitmap words
    constexpr int WPL = KW / 64;              // bitmap words per lane (contiguous)
    static_assert(CH % 4 == 0 && 64 % PIECES == 0, "whole 16-byte pieces");
    static_assert(kPickSetMaxU <= 65536 && kPickSetMaxK <= 65536, "16-bit ids and slots");
    __shared__ float xs_all[4][CH * RS];
    __shared__ float cs_all[4][CH * RS];
    __shared__ uint16_t sl_all[4][E * 64];           // [candidate][lane]: id, then slot
    __shared__ uint16_t uid_all[4][kPickSetMaxU];    // slot -> centroid id
    __shared__ unsigned long long bits_all[4][KW];   // the wave's candidate ids
    __shared__ uint16_t wb_all[4][KW];               // slots before each bitmap word
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *xs = xs_all[wave], *cs = cs_all[wave];
    uint16_t *sl = sl_all[wave], *uid = uid_all[wave], *wb = wb_all[wave];
    unsigned long long *bits = bits_all[wave];
    const int64_t p0 = ((int64_t)blockIdx.x * 4 + wave) * 64;
    if (p0 >= a.nq) return;  // whole waves only: every lane below stays to the end
    auto point = [&](int64_t s) -> int64_t { return a.order ? (int64_t)a.order[s] : a.slot0 + s; };
    const bool live = p0 + lane < a.nq;
    const int64_t qg = point(live ? p0 + lane : p0);  // lanes past the end mirror the first point
    const int kw = (int)((a.nrows + 63) / 64);         // bitmap words in use (<= KW)
#pragma unroll
    for (int i = 0; i < WPL; ++i) bits[lane * WPL + i] = 0ull;
    lds_wave_sync();
    float vmin = VS_INF, seg_bound = VS_INF;
    bool over = false;
    const int ne = pick_candidates<E>(a, qg, &vmin, &seg_bound, &over, [&](int e, int id) {
        sl[e * 64 + lane] = (uint16_t)id;
        atomicOr(&bits[id >> 6], 1ull << (id & 63));
    });
    lds_wave_sync();
    // slots: lane l ranks words [l WPL, (l + 1) WPL) after the words of the
    // lanes below it
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < WPL; ++i)
        cnt += lane * WPL + i < kw ? __popcll(bits[lane * WPL + i]) : 0;
    int incl = cnt;
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    const int u = __shfl(incl, 63);  // distinct candidates of the wave
    if (u <= kPickSetMaxU) {
        int slot = incl - cnt;
#pragma unroll
        for (int i = 0; i < WPL; ++i) {
            const int w = lane * WPL + i;
            wb[w] = (uint16_t)slot;
            unsigned long long m = w < kw ? bits[w] : 0ull;
            while (m) {
                const int b = __ffsll((long long)m) - 1;
                m &= m - 1;
                uid[slot++] = (uint16_t)(w * 64 + b);
            }
        }
    } else {
        over = true;  // (uniform: the whole wave goes to the exhaustive kernel)
    }
    lds_wave_sync();
    int emax = live && !over ? ne : 0;
    for (int o = 32; o > 0; o >>= 1) emax = max(emax, __shfl_xor(emax, o));
    for (int e = 0; e < ne && e < emax; ++e) {
        const int id = sl[e * 64 + lane];
        const unsigned long long below = bits[id >> 6] & ((1ull << (id & 63)) - 1ull);
        sl[e * 64 + lane] = (uint16_t)(wb[id >> 6] + __popcll(below));
    }
    lds_wave_sync();

    const int prow = lane / PIECES, pcol = (lane % PIECES) * 4;  // this lane's load piece
    const int nb = emax > 0 ? u : 0;  // distinct centroids to stage
    double sc[E], xx = 0.0;
#pragma unroll
    for (int e = 0; e < E; ++e) sc[e] = 0.0;
    // the points' chunk c0 (with_points) and the chunks of distinct
    // centroids b0 .. b0 + 63 (rows past u read centroid 0) into registers
    auto load = [&](int64_t c0, int b0, bool with_points, float4 (&pv)[PIECES],
                    float4 (&cv)[PIECES]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int r = i * ROWS_PER + prow;
            if (with_points) {
                const int64_t pr = point(p0 + r < a.nq ? p0 + r : p0);
                pv[i] = *(const float4 *)(a.pts + pr * a.ld + c0 + pcol);
            }
            const int id = b0 + r < nb ? uid[b0 + r] : 0;
            cv[i] = *(const float4 *)((const float *)a.xb + (int64_t)id * a.ld + c0 + pcol);
        }
    };
    // registers -> dimension-major LDS
    auto stage = [&](bool with_points, const float4 (&pv)[PIECES], const float4 (&cv)[PIECES])
                     __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int r = i * ROWS_PER + prow;
            if (with_points) {
                xs[(pcol + 0) * RS + r] = pv[i].x;
                xs[(pcol + 1) * RS + r] = pv[i].y;
                xs[(pcol + 2) * RS + r] = pv[i].z;
                xs[(pcol + 3) * RS + r] = pv[i].w;
            }
            cs[(pcol + 0) * RS + r] = cv[i].x;
            cs[(pcol + 1) * RS + r] = cv[i].y;
            cs[(pcol + 2) * RS + r] = cv[i].z;
            cs[(pcol + 3) * RS + r] = cv[i].w;
        }
    };
    // every lane continues its candidates' sums in dimension order over the
    // staged chunk (centroids b0 .. b0 + 63); the first batch of a chunk
    // also reads the lane's own point values and their squares
    float xr[CH];
    auto compute = [&](int b0) __attribute__((always_inline)) {
        if (b0 == 0) {
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                xr[j] = xs[j * RS + lane];
                xx = xx + (double)xr[j] * (double)xr[j];
            }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if (e < emax) {  // uniform: every slot index stays a constant
                const int s = e < ne ? (int)sl[e * 64 + lane] - b0 : -1;
                if (s >= 0 && s < 64) {
#pragma unroll
                    for (int j = 0; j < CH; ++j) {
                        const double dd = (double)xr[j] - (double)cs[j * RS + s];
                        sc[e] = sc[e] + dd * dd;
                    }
                }
            }
        }
    };
    if (nb <= 64) {
        // one batch per chunk (the usual case): the next chunk's loads are
        // in flight while this one is summed
        float4 pv[PIECES], cv[PIECES];
        load(0, 0, true, pv, cv);
        for (int64_t c0 = 0; c0 < a.ld; c0 += CH) {
            stage(true, pv, cv);
            lds_wave_sync();
            if (c0 + CH < a.ld) load(c0 + CH, 0, true, pv, cv);
            compute(0);
            lds_wave_sync();  // xs and cs are rewritten by the next chunk
        }
    } else {
        for (int64_t c0 = 0; c0 < a.ld; c0 += CH) {
            for (int b0 = 0; b0 < nb; b0 += 64) {
                // all loads issued before the first LDS write
                float4 pv[PIECES], cv[PIECES];
                load(c0, b0, b0 == 0, pv, cv);
                stage(b0 == 0, pv, cv);
                lds_wave_sync();
                compute(b0);
                lds_wave_sync();  // xs and cs are rewritten by the next batch or chunk
            }
        }
    }
    if (!live) return;
    double best = __builtin_huge_val();
    int bid = INT_MAX;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int id = e < ne && !over ? (int)uid[sl[e * 64 + lane]] : INT_MAX;
        if (e < ne && !over && (sc[e] < best || (sc[e] == best && id < bid))) {
            best = sc[e];
            bid = id;
        }
    }
    const bool safe = !over && bid != INT_MAX &&
                      (seg_bound == VS_INF ||
                       (double)seg_bound - (double)a.bound > (best - xx) + 1e-9 * (fabs(xx) + 1.0));
    a.assign[qg] = bid == INT_MAX ? 0 : bid;
    a.best_sq[qg] = best;
    if (!safe) a.fb_list[atomicAdd(a.fb_count, 1)] = (int32_t)qg;
}

// ---------------------------------------------------------------------------
// k-means exhaustive exact argmin for points whose shortlist was not proven:
// one workgroup per point; strict '<' in centroid order (kmeans.dart:93-101).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kmeans_exhaustive_kernel(const float *__restrict__ x,
                                                                int64_t ld, int64_t d,
                                                                const float *__restrict__ cen,
                                                                int64_t K,
                                                                const int32_t *__restrict__ list,
                                                                int32_t *assign,
                                                                double *best_sq) {
    extern __shared__ __align__(16) float xs[];  // the point's row, ld values (zero past d)
    __shared__ double dsh[256];
    __shared__ int ish[256];
    const int64_t p = list[blockIdx.x];
    for (int64_t j = threadIdx.x; j < ld; j += 256) xs[j] = x[p * ld + j];
    __syncthreads();
    double best = __builtin_huge_val();
    int bid = INT_MAX;
    // one centroid per thread; its row is read in 16-byte pieces and summed
    // in dimension order (the zero padding past d adds +0.0)
    for (int64_t c = threadIdx.x; c < K; c += 256) {
        const float4 *cc = (const float4 *)(cen + c * ld);
        double s = 0.0;
#pragma unroll 4
        for (int64_t j4 = 0; j4 < ld / 4; ++j4) {
            const float4 cv = cc[j4];
            const float4 xv = ((const float4 *)xs)[j4];
            const double d0 = (double)xv.x - (double)cv.x, d1 = (double)xv.y - (double)cv.y;
            const double d2 = (double)xv.z - (double)cv.z, d3 = (double)xv.w - (double)cv.w;
            s = s + d0 * d0;
            s = s + d1 * d1;
            s = s + d2 * d2;
            s = s + d3 * d3;
        }
        if (s < best) {  // c increases: keeps the lowest id among equals
            best = s;
            bid = (int)c;
        }
    }
    dsh[threadIdx.x] = best;
    ish[threadIdx.x] = bid;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const double v1 = dsh[threadIdx.x + s];
            const int i1 = ish[threadIdx.x + s];
            if (v1 < dsh[threadIdx.x] || (v1 == dsh[threadIdx.x] && i1 < ish[threadIdx.x])) {
                dsh[threadIdx.x] = v1;
                ish[threadIdx.x] = i1;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        assign[p] = ish[0];
        best_sq[p] = dsh[0];
    }
}

hipError_t launch_kmeans_exhaustive(const float *x, int64_t ld, int64_t d, const float *cen,
                                    int64_t K, const int32_t *list, int64_t m, int32_t *assign,
                                    double *best_sq, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    kmeans_exhaustive_kernel<<<dim3((unsigned)m), dim3(256), (size_t)ld * 4, st>>>(
        x, ld, d, cen, K, list, assign, best_sq);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k-means update: per centroid c and dimension j, the fp32 running sum over
// the cluster's points in increasing point order, then fp32(sum * fp64
// 1/count) (kmeans.dart:107-126).  `order` lists point ids grouped by
// cluster, ascending within a cluster.  One workgroup per centroid.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kmeans_update_kernel(const float *__restrict__ x,
                                                            int64_t ld, int64_t d,
                                                            const int32_t *__restrict__ order,
                                                            const int32_t *__restrict__ offsets,
                                                            const int32_t *__restrict__ counts,
                                                            int64_t min_points,
                                                            float *__restrict__ cen_out) {
    const int64_t c = blockIdx.x;
    const int cnt = counts[c];
    if (cnt < min_points) return;
    const int off = offsets[c];
    const double inv = 1.0 / (double)cnt;
    for (int64_t j = threadIdx.x; j < d; j += blockDim.x) {
        // the points' values are loaded eight at a time (independent loads
        // in flight together), then added one by one in point order
        float s = 0.0f;
        int t = 0;
        for (; t + 8 <= cnt; t += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = x[(int64_t)order[off + t + u] * ld + j];
#pragma unroll
            for (int u = 0; u < 8; ++u) s = s + v[u];
        }
        for (; t < cnt; ++t) s = s + x[(int64_t)order[off + t] * ld + j];
        cen_out[c * d + j] = (float)((double)s * inv);
    }
}

hipError_t launch_kmeans_update(const float *x, int64_t ld, int64_t d, int64_t n,
                                const int32_t *order, const int32_t *offsets, int64_t K,
                                const int32_t *counts, int64_t min_points, float *cen_out,
                                hipStream_t st) {
    (void)n;
    if (K <= 0) return hipSuccess;
    kmeans_update_kernel<<<dim3((unsigned)K), dim3(256), 0, st>>>(x, ld, d, order, offsets, counts,
                                                                  min_points, cen_out);
    return hipGetLastError();
}

// cluster sizes (integer atomics: order-independent)
__global__ void kmeans_count_kernel(const int32_t *__restrict__ assign, int64_t n,
                                    int32_t *counts) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) atomicAdd(&counts[assign[i]], 1);
}

// The same with a histogram per workgroup in LDS (K counters): each of the
// few workgroups counts a contiguous range of the points with LDS atomics
// and adds its nonzero counters to the global ones, so each global counter
// takes one atomic per workgroup instead of one per point.
__global__ __launch_bounds__(256) void kmeans_count_lds_kernel(const int32_t *__restrict__ assign,
                                                               int64_t n, int K, int32_t *counts) {
    extern __shared__ int hist[];
    for (int c = threadIdx.x; c < K; c += 256) hist[c] = 0;
    __syncthreads();
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * per, i1 = min(n, i0 + per);
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) atomicAdd(&hist[assign[i]], 1);
    __syncthreads();
    for (int c = threadIdx.x; c < K; c += 256)
        if (hist[c]) atomicAdd(&counts[c], hist[c]);
}

hipError_t launch_kmeans_count(const int32_t *assign, int64_t n, int64_t K, int32_t *counts,
                               hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (K <= 16384) {
        const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(256, (n + 8191) / 8192));
        kmeans_count_lds_kernel<<<dim3((unsigned)blocks), dim3(256), (size_t)K * 4, st>>>(
            assign, n, (int)K, counts);
    } else {
        kmeans_count_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(assign, n,
                                                                                     counts);
    }
    return hipGetLastError();
}

// Chunk of each point of a walk order: key[j] = c for order[j] in
// [n c / nchunk, n (c + 1) / nchunk) (a stable sort by these keys puts each
// chunk's points, in walk order, at that same range).
__global__ void chunk_keys_kernel(const int32_t *__restrict__ order, int64_t n, int nchunk,
                                  int32_t *key) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const int64_t v = order[j];
    int c = 0;
    for (int t = 1; t < nchunk; ++t) c += v >= n * t / nchunk ? 1 : 0;
    key[j] = c;
}

hipError_t launch_chunk_keys(const int32_t *order, int64_t n, int nchunk, int32_t *key,
                             hipStream_t st) {
    if (n <= 0) return hipSuccess;
    chunk_keys_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(order, n, nchunk,
                                                                               key);
    return hipGetLastError();
}

// How far each centroid moved between two steps: one wave per centroid, an
// upper bound on the Euclidean distance |new_c - old_c| (fp64 sum of the
// squared differences, any order, times 1 + 1e-9; +inf when not finite).
__global__ __launch_bounds__(256) void kmeans_shift_kernel(const float *__restrict__ old_cen,
                                                           int64_t ld,
                                                           const float *__restrict__ new_cen,
                                                           int64_t d, int64_t K, double *shift) {
    const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (c >= K) return;
    double s = 0.0;
    for (int64_t j = lane; j < d; j += 64) {
        const double t = (double)new_cen[c * d + j] - (double)old_cen[c * ld + j];
        s += t * t;
    }
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) shift[c] = isfinite(s) ? sqrt(s) * (1.0 + 1e-9) : (double)VS_INF;
}

hipError_t launch_kmeans_shift(const float *old_cen, int64_t ld, const float *new_cen, int64_t d,
                               int64_t K, double *shift, hipStream_t st) {
    if (K <= 0) return hipSuccess;
    kmeans_shift_kernel<<<dim3((unsigned)((K + 3) / 4)), dim3(256), 0, st>>>(old_cen, ld, new_cen,
                                                                              d, K, shift);
    return hipGetLastError();
}

// Starting values of the assign scan's running minima from the previous
// step: point i was assigned centroid c at squared distance best_sq[i], and
// c has since moved by at most shift[c], so (triangle inequality) its new
// squared distance is at most (sqrt(best_sq) + shift)^2; in the scan's
// accumulator space (|c|^2 - 2 x.c = squared distance - |x|^2, within
// `bound` of the accumulator) that is at most
//   (sqrt(best_sq) + shift)^2 (1 + 1e-9) - qnorm^2 (1 - 1e-6) + bound,
// rounded up to fp32 (qnorm is |x| rounded to fp32).  Rows i >= n (query
// padding) and anything not finite start at +inf (no bound).
__global__ void kmeans_init_kernel(const int32_t *__restrict__ assign,
                                   const double *__restrict__ best_sq,
                                   const double *__restrict__ shift,
                                   const float *__restrict__ qnorm, int64_t n, int64_t n_pad,
                                   int64_t K, float bound, const float *dev_bound, float *init) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_pad) return;
    if (dev_bound) bound = *dev_bound;
    float f = VS_INF;
    if (i < n) {
        const int32_t c = assign[i];
        const double b = best_sq[i];
        if (c >= 0 && c < K && b >= 0.0 && isfinite(b)) {
            const double r = sqrt(b) + shift[c];
            const double qn = (double)qnorm[i];
            const double v = r * r * (1.0 + 1e-9) - qn * qn * (1.0 - 1e-6) + (double)bound;
            if (isfinite(v) && v < 1e37) {
                f = (float)v;
                if ((double)f < v)  // the next float up
                    f = f == 0.f ? __uint_as_float(1u)
                                 : __uint_as_float(f > 0.f ? __float_as_uint(f) + 1u
                                                           : __float_as_uint(f) - 1u);
            }
        }
    }
    init[i] = f;
}

hipError_t launch_kmeans_init(const int32_t *assign, const double *best_sq, const double *shift,
                              const float *qnorm, int64_t n, int64_t n_pad, int64_t K, float bound,
                              const float *dev_bound, float *init, hipStream_t st) {
    if (n_pad <= 0) return hipSuccess;
    kmeans_init_kernel<<<dim3((unsigned)((n_pad + 255) / 256)), dim3(256), 0, st>>>(
        assign, best_sq, shift, qnorm, n, n_pad, K, bound, dev_bound, init);
    return hipGetLastError();
}

// The k-means accumulator bound from the largest centroid norm (cmax, on the
// device) and the largest point norm pmax: 1.25 (2 r pmax sqrt(cmax) +
// gam (cmax + 2 pmax sqrt(cmax))) + 1e-6, in fp64, rounded to fp32.
__global__ void kmeans_bound_kernel(const float *cmax, double pmax, double r, double gam,
                                    float *bound) {
    if (threadIdx.x != 0) return;
    const double c = (double)*cmax;
    const double pc = pmax * sqrt(c);
    *bound = (float)(1.25 * (2.0 * r * pc + gam * (c + 2.0 * pc)) + 1e-6);
}

hipError_t launch_kmeans_bound(const float *cmax, double pmax, double r, double gam, float *bound,
                               hipStream_t st) {
    kmeans_bound_kernel<<<dim3(1), dim3(64), 0, st>>>(cmax, pmax, r, gam, bound);
    return hipGetLastError();
}

// Exclusive prefix sums of the cluster counts (the first point of every
// cluster in the grouped order): one workgroup walks the counts in tiles of
// 1024, carrying the running total.
__global__ __launch_bounds__(1024) void exclusive_scan_i32_kernel(const int32_t *in, int64_t n,
                                                                  int32_t *out) {
    __shared__ int32_t part[1024];
    int32_t carry = 0;
    for (int64_t t0 = 0; t0 < n; t0 += 1024) {
        const int64_t i = t0 + threadIdx.x;
        const int32_t v = i < n ? in[i] : 0;
        part[threadIdx.x] = v;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {  // inclusive Hillis-Steele scan
            const int32_t add = threadIdx.x >= (unsigned)o ? part[threadIdx.x - o] : 0;
            __syncthreads();
            part[threadIdx.x] += add;
            __syncthreads();
        }
        if (i < n) out[i] = carry + part[threadIdx.x] - v;
        carry += part[1023];
        __syncthreads();
    }
}

hipError_t launch_exclusive_scan_i32(const int32_t *in, int64_t n, int32_t *out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    exclusive_scan_i32_kernel<<<dim3(1), dim3(1024), 0, st>>>(in, n, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Range search support
// ---------------------------------------------------------------------------
// Acceptance bounds in accumulator space.  acc approximates
//   L2: xn - 2 q.x = score - |q|^2      IP: -q.x = -score
// with |acc - exact| <= err(q) = c * |q| * max|x| (+ the norm rounding for
// L2).  The scan keeps acc <= athr, athr = exact bound + err, and the exact
// fp64 re-test decides.
__global__ void range_bounds_kernel(const float *__restrict__ qnorm, int64_t nq, int metric,
                                    double radius, float xmax, float rel, float *athr) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nq) return;
    const double qn = qnorm[i];
    const double xm = xmax;
    const double err =
        metric == 0 ? (double)rel * (2.0 * qn * xm + qn * qn + xm * xm) : (double)rel * qn * xm;
    double t;
    if (metric == 0)
        t = radius - qn * qn + err;
    else
        t = -radius + err;
    athr[i] = (float)t + fabsf((float)t) * 1e-6f + 1e-30f;
}

hipError_t launch_range_bounds(const PreparedQueries &pq, int64_t d, int metric, double radius,
                               float xnorm_max, int exact_q, int exact_x, int coarse, float *athr,
                               hipStream_t st) {
    if (pq.nq <= 0) return hipSuccess;
    // relative error of the split-bf16 dot product with fp32 accumulation:
    // products: each operand within 2^-16 relative of its value (hi + lo),
    // 2^-8 when a query is rounded to one bf16 plane; accumulation: npass d
    // + 1 terms, each rounding at most one unit of a truncating fp32
    // accumulator (2^-23), npass the MFMA passes (rows hi [, lo] x query
    // plane 0 [, rows hi x plane 1]), taken twice for margin.  One-pass
    // selection rounds both operands to bf16 (2^-9 each, taken four times
    // for margin).
    const int npass = coarse ? 1 : (exact_x ? 1 : 2) + (exact_q ? 0 : 1);
    double rel = 2.0 * ((double)npass * (double)d + 4.0) / 8388608.0 + 1.0 / 1048576.0;
    if (!exact_x) rel += 4.0 / 65536.0;
    if (!exact_q) rel += 4.0 / 65536.0;
    if (coarse) rel += 4.0 / 256.0;
    range_bounds_kernel<<<dim3((unsigned)((pq.nq + 255) / 256)), dim3(256), 0, st>>>(
        pq.qnorm, pq.nq, metric, radius, xnorm_max, (float)rel, athr);
    return hipGetLastError();
}

template <int ST>
__global__ void range_refine_kernel(const void *xb, int64_t ld, int64_t d, int metric,
                                    const float *__restrict__ qf, const int32_t *__restrict__ cq,
                                    const int32_t *__restrict__ ci, int64_t m, double radius,
                                    float *__restrict__ out_s, uint8_t *__restrict__ keep,
                                    int64_t nrows, int64_t nq, uint32_t *flags) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= m) return;
    const int64_t q = cq[t], id = ci[t];
    if (q < 0 || q >= nq || id < 0 || id >= nrows) {
        atomicOr(flags, kFlagBadId);
        out_s[t] = 0.f;
        keep[t] = 0;
        return;
    }
    const float *qrow = qf + q * d;
    double s = 0.0;
    for (int64_t j = 0; j < d; ++j) {
        const double xv = ST == 1 ? (double)bf16_to_f32(((const uint16_t *)xb)[id * ld + j])
                                  : (double)((const float *)xb)[id * ld + j];
        const double qv = (double)qrow[j];
        if (metric == 0) {
            const double diff = qv - xv;
            s = s + diff * diff;
        } else {
            s = s + qv * xv;
        }
    }
    out_s[t] = (float)s;
    keep[t] = metric == 0 ? (s <= radius) : (s >= radius);
}

hipError_t launch_range_refine(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                               const float *qf, const int32_t *cq, const int32_t *ci, int64_t m,
                               double radius, float *out_s, uint8_t *keep, int64_t nrows,
                               int64_t nq, uint32_t *flags, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    const dim3 grid((unsigned)((m + 255) / 256)), block(256);
    if (storage == 1)
        range_refine_kernel<1><<<grid, block, 0, st>>>(xb, ld, d, metric, qf, cq, ci, m, radius,
                                                       out_s, keep, nrows, nq, flags);
    else
        range_refine_kernel<0><<<grid, block, 0, st>>>(xb, ld, d, metric, qf, cq, ci, m, radius,
                                                       out_s, keep, nrows, nq, flags);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void max_reduce_kernel(const float *__restrict__ x, int64_t n,
                                                         float *out) {
    __shared__ float wm[4];
    float m = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        m = fmaxf(m, x[i]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    // one atomic per workgroup (the values are >= 0: their bits order as
    // unsigned integers)
    if (threadIdx.x == 0)
        atomicMax((unsigned int *)out,
                  __float_as_uint(fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]))));
}

hipError_t launch_max_reduce(const float *x, int64_t n, float *out, hipStream_t st) {
    hipError_t e = launch_fill32(out, 1, 0u, st);
    if (e != hipSuccess || n <= 0) return e;
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(1024, (n + 4095) / 4096));
    max_reduce_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, n, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Plain device copy (16-byte vector loads and stores, grid-stride), the
// yardstick for the memory counters: its bytes moved are known exactly.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void copy16_kernel(const u32x4_t *__restrict__ src,
                                                     u32x4_t *__restrict__ dst, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16;
         i += (int64_t)gridDim.x * 256)
        dst[i] = src[i];
}

hipError_t launch_copy16(const void *src, void *dst, int64_t n16, hipStream_t st) {
    if (n16 <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 256 * 32);
    copy16_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const u32x4_t *)src,
                                                                (u32x4_t *)dst, n16);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Measured-peak probes (bench support): a read-only stream of 16-byte loads
// over a buffer, and back-to-back bf16 MFMAs on registers.
// ---------------------------------------------------------------------------
// 8 independent 16-byte loads in flight per lane and step (8 KiB per wave
// step, 1 KiB contiguous per load instruction)
__global__ __launch_bounds__(256) void read16_kernel(const u32x4_t *__restrict__ src, int64_t n16,
                                                     uint32_t *out) {
    u32x4_t acc[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] = u32x4_t{0u, 0u, 0u, 0u};
    for (int64_t b = (int64_t)blockIdx.x * 2048 + threadIdx.x; b < n16;
         b += (int64_t)gridDim.x * 2048) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (b + u * 256 < n16) acc[u] ^= src[b + u * 256];
    }
    u32x4_t a = acc[0];
#pragma unroll
    for (int u = 1; u < 8; ++u) a ^= acc[u];
    const uint32_t v = a[0] ^ a[1] ^ a[2] ^ a[3];
    if (v == 0x9E3779B9u) out[0] = v;  // keeps the loads; the value is never expected
}

hipError_t launch_read16(const void *src, int64_t n16, uint32_t *out, hipStream_t st) {
    if (n16 <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n16 + 2047) / 2048, 256 * 8);
    read16_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const u32x4_t *)src, n16, out);
    return hipGetLastError();
}

// each wave: iters rounds of 8 independent v_mfma_f32_32x32x16_bf16
// (32 x 32 x 16 x 2 flop each) on register operands
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, int rnd, float *out) {
    const int lane = threadIdx.x & 63;
    // four A and four B operands; rnd: random signs and mantissas of
    // magnitude [0.5, 1) (xorshift32 per thread), else small integers
    bf16x8_t av[4], bv[4];
    uint32_t x = (blockIdx.x * 256u + threadIdx.x) * 0x9E3779B1u + 0x7F4A7C15u;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (rnd) {
                x ^= x << 13;
                x ^= x >> 17;
                x ^= x << 5;
                av[u][i] = __builtin_bit_cast(__bf16, (uint16_t)((x & 0x807Fu) | 0x3F00u));
                bv[u][i] = __builtin_bit_cast(__bf16, (uint16_t)(((x >> 16) & 0x807Fu) | 0x3F00u));
            } else {
                av[u][i] = (__bf16)(float)((lane + i + u) & 7);
                bv[u][i] = (__bf16)(float)((lane * 3 + i + u) & 7);
            }
        }
    f32x16_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) c[j][v] = 0.f;
    // the operand pair changes from one MFMA to the next (iters is even)
    for (int it = 0; it < iters; it += 2) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = mfma32_bf16(av[j & 3], bv[j >> 2], c[j]);
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = mfma32_bf16(av[j & 3], bv[2 + (j >> 2)], c[j]);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) s += c[j][v];
    if (s != s) out[0] = s;  // finite sums: never taken
}

hipError_t launch_mfma_peak(int blocks, int iters, int rnd, float *out, hipStream_t st) {
    mfma_peak_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(iters, rnd, out);
    return hipGetLastError();
}

// Chained MFMAs on given operands, one wave: the accumulation the scans
// rely on, exposed so that a test can compare every accumulator with the
// exact sum.  shape 0: v_mfma_f32_32x32x16_bf16 (M = N = 32, K-step 16);
// shape 1: v_mfma_f32_16x16x32_bf16 (M = N = 16, K-step 32).  A is
// [npass][M][K] and B [npass][N][K] bf16 bits, row-major, K = nsteps *
// K-step; C and D are [M][N] fp32.  D = C, then for each K-step s and pass p
// in that order, D += A_p[:, s] B_p[:, s]^T -- the order in which the scans
// chain their plane products (rows hi x query plane 0, rows lo x plane 0,
// rows hi x plane 1).
__global__ __launch_bounds__(64) void mfma_chain_kernel(int shape, int nsteps, int npass,
                                                        const uint16_t *__restrict__ A,
                                                        const uint16_t *__restrict__ B,
                                                        const float *__restrict__ C,
                                                        float *__restrict__ D) {
    const int lane = threadIdx.x;
    if (shape == 0) {
        const int r = lane & 31, h = lane >> 5;
        const int64_t K = (int64_t)nsteps * 16;
        f32x16_t acc;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = C[(8 * (v / 4) + 4 * h + v % 4) * 32 + r];
        for (int s = 0; s < nsteps; ++s)
            for (int p = 0; p < npass; ++p) {
                const int64_t off = ((int64_t)p * 32 + r) * K + s * 16 + 8 * h;
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(A + off));
                const bf16x8_t b = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(B + off));
                acc = mfma32_bf16(a, b, acc);
            }
#pragma unroll
        for (int v = 0; v < 16; ++v) D[(8 * (v / 4) + 4 * h + v % 4) * 32 + r] = acc[v];
    } else {
        const int r = lane & 15, g = lane >> 4;
        const int64_t K = (int64_t)nsteps * 32;
        f32x4_t acc;
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = C[(4 * g + v) * 16 + r];
        for (int s = 0; s < nsteps; ++s)
            for (int p = 0; p < npass; ++p) {
                const int64_t off = ((int64_t)p * 16 + r) * K + s * 32 + 8 * g;
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(A + off));
                const bf16x8_t b = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(B + off));
                acc = mfma_bf16(a, b, acc);
            }
#pragma unroll
        for (int v = 0; v < 4; ++v) D[(4 * g + v) * 16 + r] = acc[v];
    }
}

hipError_t launch_mfma_chain(int shape, int nsteps, int npass, const uint16_t *A,
                             const uint16_t *B, const float *C, float *D, hipStream_t st) {
    mfma_chain_kernel<<<dim3(1), dim3(64), 0, st>>>(shape, nsteps, npass, A, B, C, D);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// removeIds compaction (index_flat.dart:139-160): row r moves to
// dst_index[r] (or is dropped when -1).  One wave per row.
// ---------------------------------------------------------------------------
__global__ void compact_rows_kernel(const char *__restrict__ src, char *__restrict__ dst,
                                    const float *__restrict__ xn_src, float *__restrict__ xn_dst,
                                    const int32_t *__restrict__ dst_index, int64_t n,
                                    int64_t row_bytes) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const int64_t t = dst_index[r];
    if (t < 0) return;
    for (int64_t b = (int64_t)lane * 16; b < row_bytes; b += 64 * 16)
        *(uint4 *)(dst + t * row_bytes + b) = *(const uint4 *)(src + r * row_bytes + b);
    if (lane == 0) xn_dst[t] = xn_src[r];
}

hipError_t launch_compact_rows(const void *src, void *dst, const float *xn_src, float *xn_dst,
                               const int32_t *dst_index, int64_t n, int64_t row_bytes,
                               hipStream_t st) {
    if (n <= 0) return hipSuccess;
    compact_rows_kernel<<<dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st>>>(
        (const char *)src, (char *)dst, xn_src, xn_dst, dst_index, n, row_bytes);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic data: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11) keyed by the seed, counter = (element
// group g as 64 bits, stream as 64 bits) with g = row * groups + group, four
// values per group.  Box-Muller in fp64 on each pair of 32-bit outputs (a, b):
// u1 = ((a >> 8) + 1) 2^-24 in (0, 1], u2 = (b >> 8) 2^-24 in [0, 1),
// r = sqrt(-2 log u1), z0 = fp32(r cos(2 pi u2)), z1 = fp32(r sin(2 pi u2)).
// With normalize each row is scaled the L2NormTransform way
// (l2_norm_transform.dart:23-46): s = the fp64 sum of v * v in dimension
// order, inv = 1 / sqrt(s), o = fp32(v * inv), zero rows stay zero; bf16
// output rounds o to nearest even.  One wave per row: each lane makes its
// groups' values, and the in-order sum reads them lane by lane.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
    const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(M0, c.x), lo0 = M0 * c.x;
        const uint32_t hi1 = __umulhi(M1, c.z), lo1 = M1 * c.z;
        c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
        k.x += W0;
        k.y += W1;
    }
    return c;
}

__device__ __forceinline__ void box_muller(uint32_t a, uint32_t b, float &z0, float &z1) {
    const double u1 = ((double)(a >> 8) + 1.0) * (1.0 / 16777216.0);  // (0, 1]
    const double u2 = (double)(b >> 8) * (1.0 / 16777216.0);           // [0, 1)
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586 * u2;
    z0 = (float)(r * cos(t));
    z1 = (float)(r * sin(t));
}

__device__ __forceinline__ void gen_group(int64_t row, int64_t groups, int64_t gi, uint64_t stream,
                                          uint2 key, float z[4]) {
    const uint64_t ctr = (uint64_t)row * (uint64_t)groups + (uint64_t)gi;
    const uint4 r = philox4x32_10(make_uint4((uint32_t)ctr, (uint32_t)(ctr >> 32), (uint32_t)stream,
                                             (uint32_t)(stream >> 32)),
                                  key);
    box_muller(r.x, r.y, z[0], z[1]);
    box_muller(r.z, r.w, z[2], z[3]);
}

template <int OUT_BF16>
__global__ __launch_bounds__(256) void gen_normal_kernel(void *dst, int64_t n, int64_t d,
                                                         uint64_t seed, uint64_t stream,
                                                         int normalize) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const uint2 key = make_uint2((uint32_t)seed, (uint32_t)(seed >> 32));
    const int64_t groups = (d + 3) / 4;
    double inv = 1.0;
    if (normalize) {
        // s in dimension order: chunk c holds groups 64 c .. 64 c + 63, lane l
        // group 64 c + l; every lane adds the chunk's values lane by lane
        double s = 0.0;
        for (int64_t c0 = 0; c0 < groups; c0 += 64) {
            float z[4] = {0.f, 0.f, 0.f, 0.f};
            if (c0 + lane < groups) gen_group(row, groups, c0 + lane, stream, key, z);
            const int64_t lanes = min((int64_t)64, groups - c0);
            for (int l = 0; l < (int)lanes; ++l) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(z[u]), l));
                    if ((c0 + l) * 4 + u < d) s = s + (double)v * (double)v;
                }
            }
        }
        const double norm = sqrt(s);
        inv = norm > 0.0 ? 1.0 / norm : 0.0;
    }
    for (int64_t gi = lane; gi < groups; gi += 64) {
        float z[4];
        gen_group(row, groups, gi, stream, key, z);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t j = gi * 4 + u;
            if (j >= d) break;
            const float o = normalize ? (float)((double)z[u] * inv) : z[u];
            if (OUT_BF16)
                ((uint16_t *)dst)[row * d + j] = f32_to_bf16_rne(o);
            else
                ((float *)dst)[row * d + j] = o;
        }
    }
}

hipError_t launch_gen_normal(void *dst, int out_dtype, int64_t n, int64_t d, uint64_t seed,
                             uint64_t stream, int normalize, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 3) / 4)), block(256);
    if (out_dtype == 1)
        gen_normal_kernel<1><<<grid, block, 0, st>>>(dst, n, d, seed, stream, normalize);
    else
        gen_normal_kernel<0><<<grid, block, 0, st>>>(dst, n, d, seed, stream, normalize);
    return hipGetLastError();
}

}  // namespace vs
