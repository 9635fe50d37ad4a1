// vs_device.h -- device helpers shared by the scan kernels of libvs_hip.so.
#pragma once

#include <limits.h>

#include "vs_internal.h"

namespace vs {

#define VS_INF __builtin_huge_valf()

// Lane-group synchronisation for data exchanged through LDS or global
// memory between lanes of one wave (all waves of a workgroup share the CU's
// L1, so workgroup-scope fences order both).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Orders LDS accesses between lanes of one wave: LDS instructions of a wave
// execute in order, so only the compiler must not move them across.
__device__ __forceinline__ void lds_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// Wave-level bitonic sort of (v, i) pairs in LDS, ascending by (v, i).
// ---------------------------------------------------------------------------
__device__ inline void bitonic_sort_wave(float *sv, int *si, int n, int lane) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = lane; t < (n >> 1); t += 64) {
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
            lds_wave_sync();
        }
    }
}

struct ScanKArgs {
    const void *xb;
    int64_t ld;
    const float *xn;
    int64_t n;
    const uint16_t *qp;
    int64_t nq;
    int64_t nqblk, nsplit, rows_per_split;
    int64_t qgroup;      // GEMM-tiled scan: query blocks per XCD group
    int64_t qspc;        // GEMM-tiled scan: splits per XCD chunk
    int flush_at;        // GEMM-tiled scan: a list holding more entries is cut to kk
                         // before the next append (so its threshold keeps tightening)
    int kk, cap, metric;
    int kk_final;        // candidates the merge keeps per query
    int publish_block;   // nl * kk >= kk_final: a block's nl lists of a query bound its kk_final-th value
    float *lbound;       // per list: its own final threshold (verification of kk < kk_final)
    int32_t *list_cnt;   // per list: its entry count (lists left uncut and unpadded), or null
    float *cand_v;
    int32_t *cand_i;
    uint32_t *gthr;  // per-query threshold shared by every list (order-preserving code)
    const float *athr;
    int self_join;
    int32_t *out_q, *out_i;
    unsigned long long *count;
    int64_t out_cap;
    float kmin_margin;   // row-shared scan, k-means lists: each lane appends the values below
                         // its running minimum plus this margin
    const float *dev_bound;  // k-means lists: the bound on the device (the margin is 2.5 times
                             // it, overriding kmin_margin), or null
    const int32_t *qorder;   // k-means lists: slot s of the scan stands for point qorder[s]
                             // (s < nq; lists, counts and kmin_init stay indexed by point), or null
    const float *kmin_init;  // k-means lists: per query, a value at or above the accumulator of
                             // some scanned row (the running minimum starts there), or null
};

// Order-preserving map of finite floats to uint32 (a < b  <=>  enc(a) < enc(b)),
// so a shared threshold can be tightened with an integer atomicMin.
__device__ __forceinline__ uint32_t enc_order(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float dec_order(uint32_t u) {
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// Flush one (wave, query) list: sort, keep its kk best, set count and the
// list's own threshold, and tighten the query's shared threshold with a
// value that provably has kk_final candidates at or below it: the list's own
// kk-th value when kk == kk_final, otherwise (publish_block: nl * kk >=
// kk_final) the largest of the thresholds of the block's nl lists of this
// query.  thr_q0 points at list 0's threshold of the query; lists are bn
// apart.  Every threshold is +inf until its list has held kk entries.
__device__ inline void flush_list(float *cvq, int32_t *ciq, int *cnt_q, float *thr_q, const float *thr_q0,
                           int bn, int nl, uint32_t *gthr_q, float *sv, int *si, int cap, int kk,
                           int kk_final, int publish_block, int lane) {
    wave_sync();  // the list's global entries were appended by other lanes
    const int c = *cnt_q;
    // sort only the smallest power of two that holds the list (<= cap)
    int n = 2;
    while (n < c) n <<= 1;
    if (n > cap) n = cap;
    for (int j = lane; j < n; j += 64) {
        const bool in = j < c;
        sv[j] = in ? cvq[j] : VS_INF;
        si[j] = in ? ciq[j] : INT_MAX;
    }
    lds_wave_sync();
    bitonic_sort_wave(sv, si, n, lane);
    const int keep = c < kk ? c : kk;
    for (int j = lane; j < kk; j += 64) {
        cvq[j] = j < keep ? sv[j] : VS_INF;
        ciq[j] = j < keep ? si[j] : -1;
    }
    if (lane == 0) {
        *cnt_q = keep;
        if (c >= kk) {
            const float kth = fminf(*thr_q, sv[kk - 1]);
            *thr_q = kth;
            if (kk >= kk_final) {
                atomicMin(gthr_q, enc_order(kth));
            } else if (publish_block) {
                float b = thr_q0[0];
                for (int i = 1; i < nl; ++i) b = fmaxf(b, thr_q0[i * bn]);
                if (b < VS_INF) atomicMin(gthr_q, enc_order(b));
            }
        }
    }
    wave_sync();
}

// Cuts a wave's lists of more than `over` (>= kk) entries, one lane per list
// (lane q < bn handles list q; bn <= 64, kk <= KM): each lane keeps its
// list's kk best (value, id) pairs in registers by insertion, writes them
// back sorted, and sets and publishes the list's threshold as flush_list
// does -- the same lists and thresholds as flush_list on each of those
// lists, without visiting the lists one after another.  pad: lists of fewer
// than kk entries are padded to kk with sentinels (the final cut, over = kk).
// The block's lists of query q sit at thr[q + i tstride], i < nl (tstride 0:
// bn).
template <int KM>
__device__ __forceinline__ void cut_lists_lanes(float *cv, int32_t *ci, int *cnt_w, float *thr_w,
                                       const float *thr, int bn, int nl, uint32_t *gthr,
                                       int cap, int kk, int kk_final, int publish_block,
                                       int over, bool pad, int lane, int tstride = 0) {
    wave_sync();  // every lane's appends and counts are visible
    const int q = lane;
    if (q < bn) {
        const int c = cnt_w[q];
        const int keep = c < kk ? c : kk;
        float *cvq = cv + (int64_t)q * cap;
        int32_t *ciq = ci + (int64_t)q * cap;
        if (c > over) {
            float bv[KM];
            int bi[KM];
#pragma unroll
            for (int m = 0; m < KM; ++m) {
                bv[m] = VS_INF;
                bi[m] = INT_MAX;
            }
            // 8 entries per batch, all loaded before any is inserted (cap is
            // a multiple of 8, so a batch never leaves the list's buffer;
            // entries past the count become sentinels, which never insert)
            for (int e0 = 0; e0 < c; e0 += 8) {
                float v8[8];
                int i8[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    v8[u] = cvq[e0 + u];
                    i8[u] = ciq[e0 + u];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    float v = e0 + u < c ? v8[u] : VS_INF;
                    int id = e0 + u < c ? i8[u] : INT_MAX;
                    // insertion by (value, id); slots past kk stay +inf
#pragma unroll
                    for (int m = 0; m < KM; ++m) {
                        const bool lt = m < kk && (v < bv[m] || (v == bv[m] && id < bi[m]));
                        const float tv = lt ? bv[m] : v;
                        const int ti = lt ? bi[m] : id;
                        bv[m] = lt ? v : bv[m];
                        bi[m] = lt ? id : bi[m];
                        v = tv;
                        id = ti;
                    }
                }
            }
            float kth = VS_INF;
#pragma unroll
            for (int m = 0; m < KM; ++m) {
                if (m < kk) {
                    cvq[m] = bv[m];
                    ciq[m] = bi[m];
                }
                if (m == kk - 1) kth = bv[m];
            }
            cnt_w[q] = keep;
            thr_w[q] = fminf(thr_w[q], kth);
        } else if (pad) {
            for (int j = c; j < kk; ++j) {
                cvq[j] = VS_INF;
                ciq[j] = -1;
            }
        }
    }
    lds_wave_sync();  // the lists' thresholds are written
    if (q < bn && cnt_w[q] >= kk) {
        const float kth = thr_w[q];
        if (kk >= kk_final) {
            atomicMin(&gthr[q], enc_order(kth));
        } else if (publish_block) {
            const float *t0 = thr + q;
            const int ts = tstride ? tstride : bn;
            float b = t0[0];
            for (int i = 1; i < nl; ++i) b = fmaxf(b, t0[i * ts]);
            if (b < VS_INF) atomicMin(&gthr[q], enc_order(b));
        }
    }
    wave_sync();
}

// Word 3 of a raw buffer resource (gfx9: 32-bit data format, no swizzle).
constexpr int kBufRsrcWord3 = 0x00020000;

// 16-byte buffer load at byte voff + soff of a resource (soff uniform)
__device__ __forceinline__ u32x4_t buf_load16(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
}

__device__ __forceinline__ f32x4_t mfma_bf16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_bf16.  Lane l supplies row l % 32 of A and column
// l % 32 of B, K elements 8 * (l / 32) .. + 7 of the 16-wide K-step; it
// receives column l % 32 of D, register v holding row
// 8 * (v / 4) + 4 * (l / 32) + v % 4 (checked on gfx950 with a probe kernel
// whose D equals its row index, its column index and the sum over K).
__device__ __forceinline__ f32x16_t mfma32_bf16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Maps a flat block index to (split, query block) so that the query blocks
// of one split land on the same XCD (blocks are dealt to the 8 XCDs round-
// robin) back to back: they read the same database rows at about the same
// time and share that XCD's L2.
__device__ __forceinline__ bool map_block(int64_t nqblk, int64_t nsplit, int64_t *split,
                                          int64_t *qblk) {
    const int64_t total = nqblk * nsplit;
    const int64_t per_xcd = (total + 7) / 8;
    const int64_t w = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (w >= total) return false;
    *split = w / nqblk;
    *qblk = w % nqblk;
    return true;
}

// Grid of the GEMM-tiled scan.  The query blocks are cut into groups of qg
// consecutive blocks and the splits into runs of spc; a chunk is one group
// times one run, qg * spc workgroups (about what one XCD holds at once).
// Chunk c runs on XCD c % 8 (workgroup i runs on XCD i % 8), the chunks of
// one XCD in increasing order.  The workgroups running together on an XCD
// thus cover spc splits for qg query blocks: each database row they read is
// shared by qg workgroups through that XCD's L2, and the group's query planes
// stay resident in it.  Consecutive chunks -- the split runs of a group, or
// the groups when there is one run -- go to different XCDs, which balances
// the XCDs also when later query blocks have less work (the self-join's
// upper triangle).
__host__ __device__ inline int64_t tile_grid_space(int64_t nqblk, int64_t nsplit, int64_t qg,
                                                   int64_t spc) {
    const int64_t nch = ((nqblk + qg - 1) / qg) * ((nsplit + spc - 1) / spc);
    return ((nch + 7) / 8) * 8 * qg * spc;
}
__device__ __forceinline__ bool map_block_grouped(int64_t nqblk, int64_t nsplit, int64_t qg,
                                                  int64_t spc, int64_t *split, int64_t *qblk) {
    const int64_t nsc = (nsplit + spc - 1) / spc, cs = qg * spc;
    const int64_t nch = ((nqblk + qg - 1) / qg) * nsc;
    const int64_t i = blockIdx.x >> 3;
    const int64_t c = (i / cs) * 8 + (blockIdx.x & 7);
    if (c >= nch) return false;
    const int64_t r = i % cs;
    *split = (c % nsc) * spc + r / qg;
    *qblk = (c / nsc) * qg + r % qg;
    return *split < nsplit && *qblk < nqblk;
}

// ---------------------------------------------------------------------------
// Exact score of (query, row) in the reference's arithmetic: fp64 sum over
// j = 0..d-1 in order of q[j]*x[j] (IP) or (q[j]-x[j])^2 (L2), with the fp32
// values promoted to fp64 (index_flat.dart:78-88; index.dart:181-200).
// Rows are zero past d and so is q (qrow must hold ld values, zero past d):
// the extra terms add +0.0 to the sum.
// ---------------------------------------------------------------------------
template <int ST>
__device__ double exact_score(const float *qrow, const void *xb, int64_t ld, int64_t id,
                              int64_t d, int metric) {
    // The row and the query are read 16 elements at a time, each batch as
    // independent 16-byte loads issued before any of them is used, so that a
    // candidate costs one memory round trip per batch instead of one per
    // element pair; ld is a multiple of 64 elements and qrow (16-byte
    // aligned) holds ld values, so every load stays in bounds.  Elements past
    // d are zero in the row and in qrow: their terms are +0, and s (which
    // starts at +0 and is never -0) is unchanged by them.
    constexpr int B = 16;
    double s = 0.0;
    const int64_t dend = (d + B - 1) & ~(int64_t)(B - 1);
    for (int64_t j0 = 0; j0 < dend; j0 += B) {
        float q[B], x[B];
#pragma unroll
        for (int c = 0; c < B / 4; ++c) {
            const float4 v = *(const float4 *)(qrow + j0 + 4 * c);
            q[4 * c + 0] = v.x;
            q[4 * c + 1] = v.y;
            q[4 * c + 2] = v.z;
            q[4 * c + 3] = v.w;
        }
        if constexpr (ST == 1) {
            const uint16_t *xr = (const uint16_t *)xb + id * ld + j0;
#pragma unroll
            for (int c = 0; c < B / 8; ++c) {
                const uint4 r = *(const uint4 *)(xr + 8 * c);
                const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {  // element 2u is the low half
                    x[8 * c + 2 * u] = __builtin_bit_cast(float, w[u] << 16);
                    x[8 * c + 2 * u + 1] = __builtin_bit_cast(float, w[u] & 0xFFFF0000u);
                }
            }
        } else {
            const float *xr = (const float *)xb + id * ld + j0;
#pragma unroll
            for (int c = 0; c < B / 4; ++c) {
                const float4 v = *(const float4 *)(xr + 4 * c);
                x[4 * c + 0] = v.x;
                x[4 * c + 1] = v.y;
                x[4 * c + 2] = v.z;
                x[4 * c + 3] = v.w;
            }
        }
        if (metric == 0) {
#pragma unroll
            for (int u = 0; u < B; ++u) {
                const double diff = (double)q[u] - (double)x[u];
                s = s + diff * diff;
            }
        } else {
#pragma unroll
            for (int u = 0; u < B; ++u) s = s + (double)q[u] * (double)x[u];
        }
    }
    return s;
}

}  // namespace vs
