/*
 * vs_hip.h -- C ABI of libvs_hip.so, the MI355X (gfx950) flat exact
 * nearest-neighbour library.
 *
 * This ABI replaces, for the vector-store search path, the CUDA
 * libmat_mul.so bindings that the reference opens through dart:ffi
 * (lib/core/tensor/cuda_engine.dart:241-413, path resolution :428-455) and
 * the GpuIndexFlat slot built on them (lib/core/vector_store/gpu_index_flat.dart:40-194).
 * The reference's per-search sequence create_tensor / transpose_tensor /
 * matmul_tensors / get_tensor_data / destroy_tensor (engine.cu:94-132,328-338)
 * becomes one vs_index_search call on an HBM-resident index.
 *
 * Rules:
 *   - every size and count is int64_t; ids are int32_t because the
 *     reference's result containers are Int32List (index.dart:28-35);
 *   - every entry point returns a status (VS_OK = 0) and never fails
 *     silently; vs_last_error() returns a thread-local message for the last
 *     failing call on the calling thread;
 *   - the library owns all device memory; the caller owns host buffers
 *     except the result objects, which have their own free functions;
 *   - an index handle is single-threaded (one internal HIP stream);
 *     separate handles may be used from separate threads.  One exception:
 *     vs_index_search_device_noalloc shares one fixed scratch region per
 *     GPU between all handles, so its calls on one GPU are serialised by a
 *     per-device lock (they return only after their GPU work is done).
 */
#ifndef VS_HIP_H
#define VS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VS_API __attribute__((visibility("default")))

/* status codes */
enum {
    VS_OK = 0,
    VS_ERR_INVALID = 1,     /* bad argument: d <= 0, bad metric, k < 0, ... */
    VS_ERR_OOM = 2,         /* device or host allocation failed */
    VS_ERR_HIP = 3,         /* HIP runtime error (message holds the HIP string) */
    VS_ERR_UNSUPPORTED = 4, /* valid request outside what this build implements */
    VS_ERR_NONFINITE = 5,   /* NaN or infinity in vectors or queries */
    VS_ERR_NO_DEVICE = 6    /* no HIP device visible */
};

/* Metric codes follow the FAISDART on-disk encoding, 0 = L2, 1 = IP
 * (index_io.dart:233-243).  L2 is the squared Euclidean distance, smaller is
 * better; IP is the raw dot product, larger is better (index.dart:11-16). */
enum { VS_METRIC_L2 = 0, VS_METRIC_IP = 1 };

/* element types of caller buffers */
enum { VS_DTYPE_F32 = 0, VS_DTYPE_BF16 = 1 };

/* Storage of the database rows in HBM.
 *   F32  -- fp32, as IndexFlat's Float32List storage (index_flat.dart:20);
 *   BF16 -- bf16; fp32 input rows are rounded to nearest-even once at add;
 *   AUTO -- bf16 while every stored value is exactly a bf16 value (then
 *           results are those of fp32 storage), fp32 otherwise; the switch
 *           to fp32 happens at the first add that needs it. */
enum { VS_STORAGE_F32 = 0, VS_STORAGE_BF16 = 1, VS_STORAGE_AUTO = 2 };

typedef struct vs_index vs_index;

/* CSR range-search result, the layout of RangeSearchResult (index.dart:37-85):
 * hits of query q are [lims[q], lims[q+1]) in ascending id order. */
typedef struct vs_range_result {
    int64_t nq;
    int64_t *lims; /* nq + 1 */
    float *D;      /* lims[nq] distances (fp32 of the fp64 score) */
    int32_t *I;    /* lims[nq] ids */
} vs_range_result;

/* Pair list of a self-join, sorted by (i, j), i < j. */
typedef struct vs_pairs {
    int64_t npairs;
    int32_t *i;
    int32_t *j;
    float *s;
} vs_pairs;

/* ---- lifecycle (replaces create_tensor/destroy_tensor, engine.cu:94-107) ---- */

/* IndexFlat(d, metric) (index_flat.dart:17-18; IndexFlatL2/IP :192,196);
 * GpuIndexFlat.l2/.ip (gpu_index_flat.dart:47-51). */
VS_API int vs_index_create(int device, int64_t d, int metric, int storage, vs_index **out);
VS_API void vs_index_destroy(vs_index *idx);
/* Pre-size device storage for n vectors (avoids regrowth copies). */
VS_API int vs_index_reserve(vs_index *idx, int64_t n);
/* Drop all vectors (ntotal = 0), keep the allocation. */
VS_API int vs_index_reset(vs_index *idx);

VS_API int64_t vs_index_ntotal(const vs_index *idx);
VS_API int64_t vs_index_d(const vs_index *idx);
VS_API int vs_index_metric(const vs_index *idx);
/* Current storage (VS_STORAGE_F32 or VS_STORAGE_BF16). */
VS_API int vs_index_storage(const vs_index *idx);

/* ---- data in ---- */

/* IndexFlat.add (index_flat.dart:23-51): append n row-major host rows of d
 * elements; ids are assigned sequentially from ntotal. */
VS_API int vs_index_add(vs_index *idx, const void *xs, int src_dtype, int64_t n);
/* Same, rows already in device memory on the index's device. */
VS_API int vs_index_add_device(vs_index *idx, const void *xs_dev, int src_dtype, int64_t n);
/* IndexFlat.reconstruct (index_flat.dart:55-60) for rows [i0, i0+n) as fp32. */
VS_API int vs_index_reconstruct(vs_index *idx, int64_t i0, int64_t n, float *out);
/* IndexFlat.removeIds (index_flat.dart:139-160): drop the listed ids, compact
 * the remaining rows in order and renumber them from 0.  Ids outside
 * [0, ntotal) and duplicates are ignored, as a Set<int> lookup does. */
VS_API int vs_index_remove_ids(vs_index *idx, const int64_t *ids, int64_t n, int64_t *nremoved);

/* Loads a flat index file into a new index on `device` (storage as
 * vs_index_create): the reference's FAISDART IndexFlat blob (magic
 * 'FAISDART', version 1, kind 0x01; index_io.dart:8-26, IndexFlat.readFrom
 * index_flat.dart:176-188) or a FAISS IndexFlat blob (fourcc IxF2 / IxFI /
 * IxFl; readFaissIndex faiss_io.dart:1690-1716).  The header is parsed on
 * the host and the fp32 rows stream into HBM through a pinned staging buffer
 * of at most 64 MiB.  *is_trained (may be null) receives the header's flag.
 * Malformed headers give VS_ERR_INVALID with the reference's messages
 * ("Unknown metric code", "IndexFlat payload size ... != ntotal*d*4"). */
VS_API int vs_index_load_flat(int device, const char *path, int storage, vs_index **out,
                              int *is_trained);
/* Same from a caller's memory buffer of len bytes. */
VS_API int vs_index_load_flat_buffer(int device, const void *buf, int64_t len, int storage,
                                     vs_index **out, int *is_trained);

/* ---- search ---- */

/* IndexFlat.search (index_flat.dart:62-97) / GpuIndexFlat.search
 * (gpu_index_flat.dart:119-193).  Host queries nq x d, host outputs nq x k
 * (caller-allocated).  Rows are best-first; slots beyond ntotal hold +inf
 * (L2) or -inf (IP) with id -1 (index.dart:306-313).  Distances are the
 * fp64 sum in dimension order rounded to fp32, as the reference reports. */
VS_API int vs_index_search(vs_index *idx, const void *q, int q_dtype, int64_t nq, int64_t k,
                           float *D, int32_t *I);
/* Same with q, D and I in device memory (inputs resident in HBM).  On
 * VS_ERR_NONFINITE from bf16 queries, or from fp32 queries on an index of
 * bf16 rows, D and I hold unspecified values (their flags are read with the
 * results). */
VS_API int vs_index_search_device(vs_index *idx, const void *q_dev, int q_dtype, int64_t nq,
                                  int64_t k, float *D_dev, int32_t *I_dev);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc):
 * vs_index_search_device with every scratch buffer -- prepared queries,
 * candidate lists, thresholds, counters and the fallback paths' lists --
 * carved from one fixed region per device, a 128 MiB static device array
 * the library holds from load until the process ends.  It calls no
 * hipMalloc / hipFree / hipHostMalloc.  Limits: nq <= 64, k <= 128,
 * d <= 4096 (VS_ERR_UNSUPPORTED beyond).  Results equal those of
 * vs_index_search_device.  It is not for HIP graph capture: like every
 * search it runs on the index's own stream and synchronises it before
 * returning.  All calls on one GPU share its region, which keeps the last
 * call's contents; calls that overlap on one GPU would race on it, so a
 * per-device lock serialises them within the process. */
VS_API int vs_index_search_device_noalloc(vs_index *idx, const void *q_dev, int q_dtype,
                                          int64_t nq, int64_t k, float *D_dev, int32_t *I_dev);

/* Exact top-k of each query over subsets of the stored rows: query i scans
 * the rows ids[seg_off[i nseg + s] .. + seg_len[i nseg + s]) for s < nseg --
 * the fine scan of IndexIVFFlat.search over its probed inverted lists
 * (index_ivf_flat.dart:131-170): fp64 scores in dimension order, the k best
 * by (fp32 score, id), sentinels when fewer rows were scanned.  Host
 * buffers; any k (beyond 409 each query's subset rows are sorted on the
 * device).  An id outside [0, ntotal) gives VS_ERR_INVALID. */
VS_API int vs_index_search_subsets(vs_index *idx, const void *q, int q_dtype, int64_t nq,
                                   int64_t k, const int32_t *ids, int64_t nids,
                                   const int64_t *seg_off, const int64_t *seg_len, int64_t nseg,
                                   float *D, int32_t *I);

/* out[r] = the exact score of every stored row r against one fp32 query
 * (host, d values): l2sq / dot of index.dart:181-200 in fp64, rounded to
 * fp32 -- the closestSq refresh of the k-means++ seeding (kmeans.dart:53-84).
 * out holds ntotal floats (host). */
VS_API int vs_index_score_all(vs_index *idx, const float *q, float *out);

/* IndexFlat.rangeSearch (index_flat.dart:99-137): every stored vector with
 * dist <= radius (L2) or dot >= radius (IP), tested on the fp64 score.
 * *out is library-allocated; free it with vs_range_result_free. */
VS_API int vs_index_range_search(vs_index *idx, const void *q, int q_dtype, int64_t nq,
                                 double radius, vs_range_result **out);
VS_API void vs_range_result_free(vs_range_result *r);

/* Near-duplicate self-join over the index's own vectors: all pairs i < j
 * with dot(x_i, x_j) >= threshold (IP) or |x_i - x_j|^2 <= threshold (L2),
 * sorted by (i, j) -- the pair list bin/vector_dedup_demo.dart:115-128
 * builds from rangeSearch(all, threshold). */
VS_API int vs_index_self_join(vs_index *idx, double threshold, vs_pairs **out);
VS_API void vs_pairs_free(vs_pairs *p);

/* One Lloyd iteration of Kmeans.train (kmeans.dart:91-140) with the index's
 * vectors as the training points (metric ignored; storage must be F32):
 * assign[i] = strict-'<' argmin over centroids_in of the fp64 squared
 * distance; *obj = their fp64 sum in point order; counts[c]; centroids_out
 * = fp32 running sums in point order times fp64 1/count.  A centroid with
 * count < min_points copies the largest cluster plus (u - 0.5) * 1e-4 with
 * u taken in order from jitter_u (njitter values; the reference draws them
 * from dart:math Random).  Host buffers; centroids_out may equal centroids_in. */
VS_API int vs_kmeans_step(vs_index *points, const float *centroids_in, int64_t K,
                          int64_t min_points, const double *jitter_u, int64_t njitter,
                          int32_t *assign, float *centroids_out, int32_t *counts, double *obj);

/* ---- errors ---- */
VS_API const char *vs_last_error(void);

/* ---- bench / test support (no reference counterpart) ---- */

/* Device buffers on `device` for inputs that must be resident in HBM. */
VS_API int vs_dev_alloc(int device, int64_t bytes, void **out);
VS_API int vs_dev_free(int device, void *p);
VS_API int vs_dev_upload(int device, void *dst_dev, const void *src_host, int64_t bytes);
VS_API int vs_dev_download(int device, void *dst_host, const void *src_dev, int64_t bytes);
/* dst_dev = src_dev with a plain 16-byte-per-lane copy kernel (the yardstick
 * of the FETCH_SIZE / WRITE_SIZE counters); sizes and pointers 16-byte aligned. */
VS_API int vs_dev_copy(int device, void *dst_dev, const void *src_dev, int64_t bytes);
/* Measured peaks for the "of measured achievable" fractions: what = 0 reads
 * `bytes` (>= 1 MiB, a multiple of 16) with 16-byte loads and returns GB/s;
 * what = 1 runs register-only bf16 MFMAs (v_mfma_f32_32x32x16_bf16) on
 * every CU and returns TFLOP/s, on small-integer operands; what = 2 the same
 * on random operands (random signs and mantissas, the bit activity of real
 * data, which draws more power and lowers the sustained clock).  Best of
 * five timed runs after a warm-up. */
VS_API int vs_dev_probe(int device, int what, int64_t bytes, double *result);
/* The scans' MFMA accumulation on given operands (test support for the
 * rounding model behind the top-k exactness check): shape 0 chains
 * v_mfma_f32_32x32x16_bf16 (M = N = 32, K-step 16), shape 1
 * v_mfma_f32_16x16x32_bf16 (M = N = 16, K-step 32).  Host buffers: A
 * [npass][M][K] and B [npass][N][K] bf16 bits, K = nsteps * K-step; C and D
 * [M][N] fp32.  D = C, then for each K-step s and each pass p in order
 * D += A_p[:, s] B_p[:, s]^T.  1 <= nsteps <= 4096, 1 <= npass <= 4. */
VS_API int vs_dev_mfma_chain(int device, int shape, int64_t nsteps, int64_t npass,
                             const uint16_t *A, const uint16_t *B, const float *C, float *D);
VS_API int vs_device_count(int *count);
VS_API int vs_device_name(int device, char *buf, int64_t len);

/* Fill n x d rows at dst_dev with N(0,1) values from Philox4x32-10
 * (Salmon et al., SC'11) keyed by (seed, stream) and Box-Muller; if
 * normalize != 0 each row is then scaled by 1/sqrt(sum of squares)
 * (computed in fp64, the L2NormTransform convention,
 * l2_norm_transform.dart:23-46); out_dtype F32 or BF16 (round to nearest
 * even after normalisation). */
VS_API int vs_gen_normal(int device, void *dst_dev, int out_dtype, int64_t n, int64_t d,
                         uint64_t seed, uint64_t stream, int normalize);

/* Per-kernel timing on the index's stream with HIP events: when enabled,
 * every launch of the named kernel family is bracketed by events and its
 * duration accumulated.  Families: "scan", "merge", "range", "assign",
 * "update", "join".  Whether or not timing is enabled, the families
 * "streamed" (streaming scan, small batches; "streamed8" its eight-wave
 * form), "shared" (row-shared scan) and "gemm" (GEMM-tiled scan) count the
 * distance scans that ran on each kernel, and "gemm:S,P,WR,WQ,RB,QB,KC"
 * those of one GEMM shape (storage, query planes, row waves, query waves,
 * 32-row blocks per wave, 32-query blocks per wave, K-chunk). */
VS_API int vs_prof_enable(vs_index *idx, int on);
VS_API int vs_prof_get(vs_index *idx, const char *family, int64_t *launches, double *total_ms);
VS_API int vs_prof_reset(vs_index *idx);

/* Synchronise the index's stream. */
VS_API int vs_index_sync(vs_index *idx);

/* Test support, no counterpart in the reference: sets one planner option of
 * this handle, so that tests reach every kernel variant on small inputs.
 * The defaults are the tuned plan; every option keeps results exact.
 *   "gemm"        -1 planner rule (rows >= 256 elements, batch >= 512), 0 off, 1 any d
 *   "gemm_min_nq" smallest batch on the GEMM-tiled scan (0: the rule's)
 *   "gemm_wq", "gemm_qb", "gemm_kc"  force that GEMM shape field (0: any)
 *   "gemm4"       1: the four-wave pipelined GEMM-tiled kernel where it applies (bf16
 *                 rows, one query plane; shape 2,2,4,4,32); 0 (default): the eight-wave one
 *   "share"       -1 rule (bf16 rows of 128 elements, batch >= 256), 0 off, 1 also 256
 *   "coarse"      1: one-pass bf16 selection of fp32 rows (range, self-join, k-means)
 *   "copy16"      1: that selection reads a bf16 copy of the rows
 *   "guess"       1: large batches start from thresholds estimated on a row sample
 *   "prepass"     1: small batches seed their thresholds from a pre-pass
 *   "prepass_log2" 10..20: that pre-pass scans at least 2^value rows (default 16)
 *   "scan_kkw"    >0: per-list keep forced down (exercises the list verification)
 *   "scan_nw8"    1: eight-wave streaming scan where it fits
 *   "km16"        1: the k-means assign reads a bf16 copy of the centroids
 *   "km16_rt"     2 or 4: 16-row blocks per tile of that scan
 *   "km16_nqb"    2 or 4 (default): 16-point blocks per wave of that scan (4: 32-row tiles)
 *   "pick_order"  1: the k-means pick walks the points grouped by the last step's clusters
 *   "assign_order" 1: so does the k-means assign scan
 *   "merge_mu"    1, 2, 4 or 8: 1,024-entry list chunks the merge reads per pass (0: by
 *                 batch size)
 *   "fail_alloc"  n > 0: the n-th device allocation of any index from now on, on
 *                 this thread, fails as VS_ERR_OOM (failure-path tests; 0 clears it)
 * Unknown names and out-of-range values: VS_ERR_INVALID. */
VS_API int vs_index_set_option(vs_index *idx, const char *name, int64_t value);

#ifdef __cplusplus
}
#endif

#endif /* VS_HIP_H */
