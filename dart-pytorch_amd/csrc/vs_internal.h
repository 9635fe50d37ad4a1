// vs_internal.h -- shared definitions of libvs_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Row storage is padded so that one row is a whole number of 256-byte
// segments: the scan kernels consume rows in 64-byte K-steps, four at a time,
// without tail handling.
constexpr int64_t kRowAlignBytes = 256;
// Device row capacity is a multiple of kRowCapAlign; kRowSlack zero rows
// follow the capacity (rows past ntotal are zero too), so the last row tile
// of a scan -- at most kRowSlack rows -- may be read whole without bounds
// checks.
constexpr int64_t kRowCapAlign = 256;
constexpr int64_t kRowSlack = 512;

// ---------------------------------------------------------------------------
// bf16 helpers (round to nearest even; inputs are finite)
// ---------------------------------------------------------------------------
__host__ __device__ inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__host__ __device__ inline float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

namespace vs {

// ---------------------------------------------------------------------------
// Kernel-side argument blocks
// ---------------------------------------------------------------------------

// Prepared queries: the B operand of the distance MFMA.  For query q, plane p
// (p < planes) holds ld bf16 values at qp + (q * planes + p) * ld.  Plane 0 is
// bf16(s * q), plane 1 is bf16(s * q - plane0) with s = -2 (L2) or -1 (IP),
// so the accumulator xn - 2 q.x (L2) or -q.x (IP) is "smaller is better"
// for both metrics.  Rows beyond d and queries beyond nq are zero.
struct PreparedQueries {
    uint16_t *qp = nullptr;  // [nq_pad][planes][ld] bf16
    float *qf = nullptr;     // [nq][d] fp32 copy of the queries as given
    float *qnorm = nullptr;  // [nq] sqrt of the fp64 sum of squares
    int planes = 1;
    int64_t nq = 0, nq_pad = 0;
};

// Status flags written by the query-preparation kernel.
// kFlagBadId: a kernel met a candidate id outside the rows it indexes (an
// internal error, reported instead of reading past the rows).
enum : uint32_t { kFlagNonFinite = 1u, kFlagNotBf16 = 2u, kFlagBadId = 4u };

// order-preserving code of +inf (see enc_order in vs_kernels.hip)
constexpr uint32_t kGthrInit = 0xFF800000u;

// ---------------------------------------------------------------------------
// Launchers (vs_kernels.hip).  All enqueue on `st`; none synchronises.
// ---------------------------------------------------------------------------

// x (n rows, d elems, src dtype, src row stride in elements) -> storage rows
// (dst dtype, ld) plus xn[i] = fp32(fp64 sum of squares of the stored values).
// flags |= kFlagNonFinite / kFlagNotBf16 as found in the source values.
hipError_t launch_store_rows(const void *src, int src_dtype, int64_t src_stride, int64_t n,
                             int64_t d, void *dst, int dst_dtype, int64_t ld, float *xn,
                             uint32_t *flags, hipStream_t st);

// Build PreparedQueries from n query rows (src dtype / stride).
hipError_t launch_prepare_queries(const void *src, int src_dtype, int64_t src_stride, int64_t nq,
                                  int64_t d, int64_t ld, int metric, const PreparedQueries &pq,
                                  uint32_t *flags, hipStream_t st);

struct ScanPlan {
    int bn = 64;          // queries per block (16 * nqb)
    int tm = 2;           // 16-row blocks per wave tile
    int kk = 16;          // per-list kept candidates (power of two)
    int kk_final = 16;    // candidates kept per query by the merge (power of two, >= kk)
    int cap = 64;         // per-list buffer capacity (power of two)
    int nks = 0;          // >0: queries held in registers for this many K-steps
    int lw = 4;           // candidate lists per (workgroup, query): the workgroup's waves
    int kind = 0;         // 0: streaming scan (vs_kernels.hip);
                          // 2: GEMM-tiled scan (vs_gemm.hip); 3: row-shared scan (vs_share.hip:
                          // nks K-steps, bn = 64 * query blocks per wave, tm = 16-row blocks per tile)
    int g_wq = 2, g_qb = 4;  // GEMM-tiled scan: query waves, 32-query blocks per wave
                             // (row waves = lw, 32-row blocks per wave = tile_rb,
                             // K-chunk = tile_kc)
    int g_pipe = 0;       // GEMM-tiled scan: 1 = the four-wave pipelined kernel (bf16 rows, one
                          // query plane; shape 2 x 2 waves, 4 x 4 blocks, K-chunk 32)
    int tile_rb = 2;      // GEMM-tiled scan: 32-row blocks per wave
    int tile_kc = 32;     // GEMM-tiled scan: K-chunk per pipeline step (elements)
    int tile_st = 1, tile_pb = 1;  // GEMM-tiled and row-shared scans: storage and query planes
                                   // they were planned for
    int64_t tile_group = 8;        // GEMM-tiled scan: query blocks per XCD group (grid order)
    int64_t tile_spc = 1;          // GEMM-tiled scan: splits per XCD chunk (grid order)
    int share_topm = 0;   // row-shared scan: >0 keeps per-lane register top-m values (sample
                          // estimates; lists get 4 * m values per query and workgroup, ids 0)
    int share_kmin = 0;   // row-shared scan: k-means lists (each lane appends what lies below its
                          // running minimum + kmin_margin; a list that would fill is marked
                          // full, count cap + 1, and takes no more)
    float kmin_margin = 0.f;
    const float *dev_bound = nullptr;  // k-means: the accumulator bound on the device; when set,
                                       // the scan's and the pick's margin is 2.5 times it and
                                       // kmin_margin is ignored
    const int32_t *qorder = nullptr;   // k-means lists: the points in the order the scan walks
                                       // them (slot s: point qorder[s]), or null (index order)
    const float *kmin_init = nullptr;  // k-means lists: per query (nq_pad entries), a value at or
                                       // above the accumulator of some scanned row, or null
    int uncut = 0;        // streaming scan: lists are left uncut at the end and their entry
                          // counts written to list_cnt, as the row-shared scan's (for scans
                          // over short samples, whose lists end full)
    int merge_mu = 1;     // merge: 1024-entry chunks each workgroup loads per pass (1, 2, 4, 8;
                          // more hides load latency when few queries leave most CUs idle)
    int merge_g = 1;      // merge: workgroups per query.  > 1: each reduces a slice of the
                          // query's lists to its kk_final best pairs, written to a partial
                          // area right after the lists ([nqblk bn][merge_g][kk_final]), and
                          // a second pass merges those (small batches over many lists)
    int64_t nqblk = 0;    // query blocks
    int64_t nsplit = 0;   // database splits
    int64_t rows_per_split = 0;
    size_t lds_bytes = 0;
};

// Top-k scan: per (query block, split, wave) lists of the kk best approximate
// candidates, written to cand_v / cand_i ([nqblk][nsplit][lw][bn][cap]).
// gthr [nq_pad] holds each query's shared threshold in an order-preserving
// uint32 code; it must start at the code of +inf (kGthrInit).  The row-shared
// scan (kind 3) leaves its lists uncut and writes their entry counts to
// list_cnt ([nqblk][nsplit][lw][bn], then the largest count, which must start
// at 0; required for that kind, others ignore it).
hipError_t launch_scan_topk(const void *xb, int storage, int64_t ld, const float *xn, int64_t n,
                            int metric, const PreparedQueries &pq, const ScanPlan &plan,
                            float *cand_v, int32_t *cand_i, uint32_t *gthr, float *lbound,
                            int32_t *list_cnt, hipStream_t st);

// Exactness check of a top-k merge: the largest stored row norm and the
// accumulator's error model (relative error err_r of one product of MFMA
// operands, accumulation factor err_g); queries whose selection cannot be
// proven exact are appended to vx_list (count in *vx_count).
struct TopkCheck {
    float xmax = 0.f;
    float err_r = 0.f;
    float err_g = 0.f;
    int32_t *vx_count = nullptr;
    int32_t *vx_list = nullptr;
};

// Merge the per-wave lists of each query, re-rank the kk survivors with the
// exact fp64 distance and write the k best (sentinel-filled) to D / I.
// Queries the merge cannot prove exact are appended to vf_list (count in
// *vf_count): lists shortened below kk_final (lbound non-null) or, when
// guess != 0, fewer than kk_final candidates found below an estimated
// threshold.  With plan.merge_g > 1 the buffers continue past the lists with
// the partial area (nqblk bn merge_g kk_final entries), which it overwrites.
hipError_t launch_merge_refine(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                               const PreparedQueries &pq, const ScanPlan &plan,
                               float *cand_v, int32_t *cand_i, const uint32_t *gthr,
                               const float *lbound, int32_t *vf_count, int32_t *vf_list,
                               int64_t k, float *D, int32_t *I, int64_t nrows, uint32_t *flags,
                               int guess, const int32_t *list_cnt, const TopkCheck *chk,
                               hipStream_t st);

// Exact top-kk lists of nq queries (fp32 rows qf [nq][d]): rows of split s
// are [s * rows_per_split, ...); lists cand_v / cand_i [nq][nsplit][kk] hold
// (fp32 key, id), key = score (L2) or -score (IP), sentinels (+inf, -1).
// kk: a multiple of 4 in [4, 512].
// With ids non-null, list (q, s) covers the rows ids[seg_off[q nsplit + s]
// .. + seg_len[q nsplit + s]) instead of a split (ids outside [0, n) set
// kFlagBadId in *flags and are skipped).
hipError_t launch_exact_lists(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                              const float *qf, int64_t nq, int64_t n, int kk, int64_t nsplit,
                              int64_t rows_per_split, float *cand_v, int32_t *cand_i,
                              hipStream_t st, const int32_t *ids = nullptr,
                              const int64_t *seg_off = nullptr, const int64_t *seg_len = nullptr,
                              uint32_t *flags = nullptr);

// out[r] = fp32 of the exact fp64 score of each of the n rows against the
// fp32 query qf[d] (L2: squared distance, IP: dot).
hipError_t launch_exact_all(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                            const float *qf, int64_t n, float *out, hipStream_t st);

// Row gather / scatter of w 32-bit words per row by an index list, and a
// 32-bit fill.
hipError_t launch_gather_rows(const void *src, const int32_t *list, int64_t m, int64_t w,
                              void *dst, hipStream_t st);
hipError_t launch_scatter_rows(const void *src, const int32_t *list, int64_t m, int64_t w,
                               void *dst, hipStream_t st);
hipError_t launch_fill32(void *p, int64_t n, uint32_t v, hipStream_t st);

// Exact top-k by sorting (any k): for nq queries (fp32 rows qf [nq][d]) the
// fp64 score of every row, as keys (fp32 key code, id), sorted per query;
// D / I [nq][k] receive the k first, sentinel-filled past n.  keys holds
// qchunk * n + n words of 64 bits, tmp tmp_bytes (query with tmp == nullptr).
hipError_t exact_sort_topk(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                           const float *qf, int64_t nq, int64_t n, int64_t k, float *D, int32_t *I,
                           uint64_t *keys, int64_t qchunk, void *tmp, size_t &tmp_bytes,
                           hipStream_t st);
// The same for one query (fp32 row qf [d]) over the rows ids[0 .. m) (ids in
// [0, ntotal), checked by the caller): keys holds 2 m words of 64 bits, tmp
// tmp_bytes (query with tmp == nullptr); D / I [k], sentinel-filled past m.
hipError_t exact_sort_topk_ids(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                               const float *qf, const int32_t *ids, int64_t m, int64_t k, float *D,
                               int32_t *I, uint64_t *keys, void *tmp, size_t &tmp_bytes,
                               hipStream_t st);

// Threshold seeding from a pre-pass scan: every query's shared threshold
// (gthr) is tightened to one code above the seed_rank-th (0: kk_final-th)
// smallest accumulator value its lists hold (partial area as for
// launch_merge_refine).
hipError_t launch_merge_threshold(const PreparedQueries &pq, const ScanPlan &plan,
                                  float *cand_v, int32_t *cand_i, uint32_t *gthr,
                                  int64_t ld, int seed_rank, const int32_t *list_cnt,
                                  hipStream_t st);

// Range scan: appends (query, id) of every approximate score within the
// per-query acceptance bound athr (accumulator space) to out_q / out_i
// (capacity cap); *count receives the total number found (may exceed cap).
// If self_join, only ids > query index are considered and query q is row
// q of the database.
hipError_t launch_scan_range(const void *xb, int storage, int64_t ld, const float *xn, int64_t n,
                             const PreparedQueries &pq, const ScanPlan &plan, const float *athr,
                             int self_join, int metric, int32_t *out_q, int32_t *out_i,
                             unsigned long long *count, int64_t cap, hipStream_t st);

// Exact fp64 re-test of range candidates: s = fp64 score of (q, id); keep[j]
// = s <= radius (L2) or s >= radius (IP); out_s[j] = fp32(s).
hipError_t launch_range_refine(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                               const float *qf, const int32_t *cq, const int32_t *ci, int64_t m,
                               double radius, float *out_s, uint8_t *keep, int64_t nrows,
                               int64_t nq, uint32_t *flags, hipStream_t st);

// Per-query acceptance bounds for the range scan (accumulator space).
hipError_t launch_range_bounds(const PreparedQueries &pq, int64_t d, int metric, double radius,
                               float xnorm_max, int exact_q, int exact_x, int coarse, float *athr,
                               hipStream_t st);

// Measured-peak probes: n16 16-byte loads (a read-only stream), and blocks
// workgroups of 4 waves each running iters rounds of 8 independent
// 32x32x16 bf16 MFMAs (out: a word the kernels leave unwritten).
hipError_t launch_read16(const void *src, int64_t n16, uint32_t *out, hipStream_t st);
hipError_t launch_mfma_peak(int blocks, int iters, int rnd, float *out, hipStream_t st);
hipError_t launch_mfma_chain(int shape, int nsteps, int npass, const uint16_t *A,
                             const uint16_t *B, const float *C, float *D, hipStream_t st);

// dst = src, n16 16-byte words (both 16-byte aligned)
hipError_t launch_copy16(const void *src, void *dst, int64_t n16, hipStream_t st);

// max over rows of xn (for margins)
hipError_t launch_max_reduce(const float *x, int64_t n, float *out, hipStream_t st);

// Compact database rows: keep rows whose flag is 0, in order.
hipError_t launch_compact_rows(const void *src, void *dst, const float *xn_src, float *xn_dst,
                               const int32_t *dst_index, int64_t n, int64_t row_bytes,
                               hipStream_t st);

// k-means update helpers
hipError_t launch_kmeans_update(const float *x, int64_t ld, int64_t d, int64_t n,
                                const int32_t *order, const int32_t *offsets, int64_t K,
                                const int32_t *counts, int64_t min_points, float *cen_out,
                                hipStream_t st);

// Exact fp64 argmin over a shortlist; flags points whose shortlist cannot be
// proven to contain the argmin (then the caller runs the exhaustive path).
hipError_t launch_kmeans_pick(const float *x, int64_t ld, int64_t d, int64_t n, const float *cen,
                              int64_t K, const float *cand_v, const int32_t *cand_i,
                              const uint32_t *gthr, const ScanPlan &plan, float bound,
                              const float *qf, int32_t *assign,
                              double *best_sq, int32_t *fallback_count, int32_t *fallback_list,
                              uint32_t *flags, const int32_t *list_cnt, const int32_t *order,
                              hipStream_t st, int64_t slot0 = 0, int64_t nslots = -1);
// (row-shared k-means lists only) slots [slot0, slot0 + nslots) of the walk:
// points order[0 .. nslots) when order is given (the caller passes the
// chunk's part of it), else points slot0 .. slot0 + nslots - 1.
hipError_t launch_chunk_keys(const int32_t *order, int64_t n, int nchunk, int32_t *key,
                             hipStream_t st);

hipError_t launch_kmeans_count(const int32_t *assign, int64_t n, int64_t K, int32_t *counts,
                               hipStream_t st);
// |new_c - old_c| per centroid (upper bounds, fp64); old rows ld apart, new dense.
hipError_t launch_kmeans_shift(const float *old_cen, int64_t ld, const float *new_cen, int64_t d,
                               int64_t K, double *shift, hipStream_t st);
// Starting values of the assign scan's running minima (kmin_init) from the
// previous step's assignments and squared distances and the centroid shifts.
hipError_t launch_kmeans_init(const int32_t *assign, const double *best_sq, const double *shift,
                              const float *qnorm, int64_t n, int64_t n_pad, int64_t K, float bound,
                              const float *dev_bound, float *init, hipStream_t st);
// *bound = the k-means accumulator bound from the largest centroid norm *cmax
// and the largest point norm pmax (fp64 arithmetic, rounded to fp32), so
// that no host round trip separates the centroids' norms from the scan.
hipError_t launch_kmeans_bound(const float *cmax, double pmax, double r, double gam, float *bound,
                               hipStream_t st);
hipError_t launch_exclusive_scan_i32(const int32_t *in, int64_t n, int32_t *out, hipStream_t st);

// Stable sort of (key, value) int32 pairs by key (rocPRIM radix sort).
// Call with tmp == nullptr to query tmp_bytes.
hipError_t sort_pairs_by_key(void *tmp, size_t &tmp_bytes, const int32_t *kin, int32_t *kout,
                             const int32_t *vin, int32_t *vout, int64_t n, int key_bits,
                             hipStream_t st);

hipError_t launch_kmeans_exhaustive(const float *x, int64_t ld, int64_t d, const float *cen,
                                    int64_t K, const int32_t *list, int64_t m, int32_t *assign,
                                    double *best_sq, hipStream_t st);

hipError_t launch_gen_normal(void *dst, int out_dtype, int64_t n, int64_t d, uint64_t seed,
                             uint64_t stream, int normalize, hipStream_t st);

// Shape rules shared by the host planner and the kernels.
int64_t storage_ld(int64_t d, int storage);  // elements per stored row
size_t scan_lds_bytes(int bn, int planes, int64_t ld, int cap, int nw);
// LDS of the merge workgroup reading mu chunks per pass
size_t merge_lds_bytes(int64_t ld, int mu);
// The built shapes of the GEMM-tiled scan, in the planner's order of
// preference: X(storage, query planes, row waves, query waves, 32-row blocks
// per wave, 32-query blocks per wave, K-chunk).  A workgroup covers
// 32 * row waves * row blocks database rows by 32 * query waves * query
// blocks queries per tile.  Storage 2 = fp32 rows read as their bf16 hi
// plane only (one-pass selection, kSelectCoarse below).
#define VS_GEMM_SHAPES(X)                                                                     \
    X(1, 1, 2, 4, 4, 2, 64)                                                                   \
    X(1, 1, 2, 2, 4, 2, 64)                                                                   \
    X(1, 1, 2, 4, 4, 2, 32)                                                                   \
    X(2, 1, 2, 4, 4, 2, 32)                                                                   \
    X(2, 1, 2, 2, 4, 2, 32)                                                                   \
    X(1, 1, 2, 2, 4, 2, 32)                                                                   \
    X(1, 2, 2, 4, 4, 2, 32)                                                                   \
    X(1, 2, 2, 2, 4, 2, 32)                                                                   \
    X(0, 2, 2, 4, 4, 2, 16)                                                                   \
    X(0, 2, 2, 2, 4, 2, 32)                                                                   \
    X(0, 1, 2, 4, 4, 2, 32)                                                                   \
    X(0, 1, 2, 2, 4, 2, 32)

// Storage code of the one-pass selection (fp32 rows, bf16 hi plane and the
// first query plane only): the GEMM-tiled scan's shapes with storage 2.
constexpr int kSelectCoarse = 2;

// LDS of the GEMM-tiled scans (stages plus list bookkeeping).
size_t gemm_lds_bytes(int st, int pb, int wr, int wq, int rb, int qb, int kc, int cap);
// LDS of the four-wave pipelined GEMM-tiled scan (four stages plus list
// bookkeeping).
size_t gemm4_lds_bytes(int cap);

// LDS of the row-shared scan (two row stages plus list bookkeeping).
size_t share_lds_bytes(int nks, int nqb, int rt, int cap, int lw);
// Row-shared scan workgroups one CU holds at once (0: no such shape; mode 0
// lists, 2 top-m values, 4 k-means lists).
int share_blocks_per_cu(int st, int nks, int bn, int rt, int64_t ld, size_t lds, int mode);
// m of the row-shared scan's register top-m variant (threshold estimates):
// values kept per lane and query.
int share_topm_est();

struct ScanKArgs;
hipError_t launch_share_scan(const ScanPlan &plan, const ScanKArgs &args, hipStream_t st);
template <int MODE>
hipError_t launch_gemm_scan(int storage, int planes, const ScanPlan &plan, const ScanKArgs &args,
                            hipStream_t st);

}  // namespace vs
