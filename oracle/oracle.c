/*
 * oracle.c -- CPU restatement of the reference's flat exact-search path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP library's
 * results are compared against (tests/, __graft_entry__.smoke(), and the
 * cpu_baseline leg of bench.py).  It is never linked into, loaded by, or
 * called from the product library; the product fails loudly when its HIP
 * build is missing instead of falling back to this code.
 *
 * The reference (KellyKinyama/dart-pytorch) is Dart and cannot be built here
 * (no Dart SDK), so each function below restates the Dart code it cites,
 * keeping its numerics:
 *   - distances are fp64 sums, in dimension order j = 0..d-1, of products /
 *     squared differences of fp32 values promoted to fp64
 *     (lib/core/vector_store/index_flat.dart:75-90, index.dart:181-200);
 *   - the k-NN heap stores fp32 scores but compares the incoming fp64 score
 *     against the stored fp32 root and accepts only strictly better scores
 *     (index.dart:213-299);
 *   - range search compares the fp64 score against the fp64 radius before the
 *     score is stored as fp32 (index_flat.dart:99-137);
 *   - k-means assignment is a strict-'<' argmin over fp64 squared distances,
 *     the objective an fp64 sum in point order, and the update fp32 running
 *     sums in point order scaled by fp64 1/count (kmeans.dart:91-140).
 *
 * Compile with -ffp-contract=off and without -ffast-math: fused multiply-add
 * contraction would change the fp64 L2 sums.  Threads split the query (or
 * point) loop only; every per-query result is computed by one thread in the
 * reference's order, so results do not depend on the thread count.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_L2 0
#define ORC_IP 1

int orc_version(void) { return 1; }

/* ------------------------------------------------------------------------ */
/* TopK: bounded binary heap, root = worst accepted (index.dart:213-331).    */
/* ------------------------------------------------------------------------ */
typedef struct {
    int64_t k;
    int max_is_worst; /* 1 = L2 (keep smallest), 0 = IP (keep largest) */
    float *score;
    int32_t *id;
    int64_t size;
} topk_t;

/* _worse(i, j) on the fp32-stored scores (index.dart:262-263). */
static inline int tk_worse(const topk_t *h, int64_t i, int64_t j) {
    return h->max_is_worst ? (h->score[i] > h->score[j]) : (h->score[i] < h->score[j]);
}

static inline void tk_swap(topk_t *h, int64_t a, int64_t b) {
    float ts = h->score[a];
    h->score[a] = h->score[b];
    h->score[b] = ts;
    int32_t ti = h->id[a];
    h->id[a] = h->id[b];
    h->id[b] = ti;
}

/* index.dart:265-280 */
static void tk_sift_up(topk_t *h, int64_t i) {
    while (i > 0) {
        int64_t p = (i - 1) >> 1;
        if (tk_worse(h, i, p)) {
            tk_swap(h, i, p);
            i = p;
        } else {
            break;
        }
    }
}

/* index.dart:282-299 */
static void tk_sift_down(topk_t *h, int64_t i) {
    int64_t n = h->size;
    for (;;) {
        int64_t l = 2 * i + 1, r = 2 * i + 2, w = i;
        if (l < n && tk_worse(h, l, w)) w = l;
        if (r < n && tk_worse(h, r, w)) w = r;
        if (w == i) break;
        tk_swap(h, i, w);
        i = w;
    }
}

/* index.dart:248-260: the incoming score is an fp64 value compared against
 * the fp32-stored root; it is stored rounded to fp32. */
static inline void tk_push(topk_t *h, double s, int32_t id) {
    if (h->size < h->k) {
        h->score[h->size] = (float)s;
        h->id[h->size] = id;
        h->size++;
        tk_sift_up(h, h->size - 1);
    } else if ((h->max_is_worst && s < (double)h->score[0]) ||
               (!h->max_is_worst && s > (double)h->score[0])) {
        h->score[0] = (float)s;
        h->id[0] = id;
        tk_sift_down(h, 0);
    }
}

typedef struct {
    float s;
    int64_t pos;
    int dir; /* +1 ascending, -1 descending */
} sort_item_t;

static int cmp_item(const void *a, const void *b) {
    const sort_item_t *x = (const sort_item_t *)a, *y = (const sort_item_t *)b;
    if (x->s != y->s) {
        int lt = x->s < y->s;
        return x->dir > 0 ? (lt ? -1 : 1) : (lt ? 1 : -1);
    }
    /* equal scores keep heap-array order: Dart's List.sort is an insertion
     * sort (stable) for lists of up to 33 elements; above that the order of
     * exactly tied scores is not pinned. */
    return (x->pos > y->pos) - (x->pos < y->pos);
}

/* index.dart:306-330: sentinels, then the heap entries sorted best-first. */
static void tk_sorted(const topk_t *h, float *D, int32_t *I, sort_item_t *tmp) {
    for (int64_t i = 0; i < h->k; i++) {
        D[i] = h->max_is_worst ? INFINITY : -INFINITY;
        I[i] = -1;
    }
    for (int64_t i = 0; i < h->size; i++) {
        tmp[i].s = h->score[i];
        tmp[i].pos = i;
        tmp[i].dir = h->max_is_worst ? 1 : -1;
    }
    qsort(tmp, (size_t)h->size, sizeof(sort_item_t), cmp_item);
    for (int64_t i = 0; i < h->size; i++) {
        D[i] = h->score[tmp[i].pos];
        I[i] = h->id[tmp[i].pos];
    }
}

/* ------------------------------------------------------------------------ */
/* Distances (index_flat.dart:78-88, index.dart:181-200, kmeans.dart:149-156) */
/* ------------------------------------------------------------------------ */
static inline double dist_ip(const float *q, const float *x, int64_t d) {
    double s = 0.0;
    for (int64_t j = 0; j < d; j++) s += (double)q[j] * (double)x[j];
    return s;
}

static inline double dist_l2(const float *q, const float *x, int64_t d) {
    double s = 0.0;
    for (int64_t j = 0; j < d; j++) {
        double diff = (double)q[j] - (double)x[j];
        s += diff * diff;
    }
    return s;
}

/* Four database rows at once: four independent sequential sums, each in the
 * same j order as the scalar loop, so the results are bit-identical to it. */
static inline void dist4(int metric, const float *q, const float *x0, int64_t d, double out[4]) {
    const float *x1 = x0 + d, *x2 = x1 + d, *x3 = x2 + d;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if (metric == ORC_L2) {
        for (int64_t j = 0; j < d; j++) {
            double qj = (double)q[j];
            double e0 = qj - (double)x0[j], e1 = qj - (double)x1[j];
            double e2 = qj - (double)x2[j], e3 = qj - (double)x3[j];
            s0 += e0 * e0;
            s1 += e1 * e1;
            s2 += e2 * e2;
            s3 += e3 * e3;
        }
    } else {
        for (int64_t j = 0; j < d; j++) {
            double qj = (double)q[j];
            s0 += qj * (double)x0[j];
            s1 += qj * (double)x1[j];
            s2 += qj * (double)x2[j];
            s3 += qj * (double)x3[j];
        }
    }
    out[0] = s0;
    out[1] = s1;
    out[2] = s2;
    out[3] = s3;
}

static inline double dist1(int metric, const float *q, const float *x, int64_t d) {
    return metric == ORC_L2 ? dist_l2(q, x, d) : dist_ip(q, x, d);
}

/* ------------------------------------------------------------------------ */
/* Thread helper                                                            */
/* ------------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, int64_t begin, int64_t end, int tid);

typedef struct {
    range_fn fn;
    void *ctx;
    int64_t begin, end;
    int tid;
} thr_arg_t;

static void *thr_main(void *p) {
    thr_arg_t *a = (thr_arg_t *)p;
    a->fn(a->ctx, a->begin, a->end, a->tid);
    return NULL;
}

/* Splits [0, n) into nthreads contiguous blocks; thread t gets block t. */
static void parallel_for(int64_t n, int nthreads, range_fn fn, void *ctx) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t)nthreads > n) nthreads = n > 0 ? (int)n : 1;
    if (nthreads == 1) {
        fn(ctx, 0, n, 0);
        return;
    }
    pthread_t th[256];
    thr_arg_t args[256];
    for (int t = 0; t < nthreads; t++) {
        args[t].fn = fn;
        args[t].ctx = ctx;
        args[t].begin = n * t / nthreads;
        args[t].end = n * (t + 1) / nthreads;
        args[t].tid = t;
        pthread_create(&th[t], NULL, thr_main, &args[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* IndexFlat.search (index_flat.dart:62-97)                                  */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *xb, *xq;
    int64_t n, d, k;
    int metric;
    float *D;
    int32_t *I;
    int err;
} search_ctx_t;

static void search_range(void *p, int64_t q0, int64_t q1, int tid) {
    (void)tid;
    search_ctx_t *c = (search_ctx_t *)p;
    int64_t k = c->k, d = c->d, n = c->n;
    topk_t h;
    h.k = k;
    h.max_is_worst = c->metric == ORC_L2;
    h.score = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
    h.id = (int32_t *)malloc(sizeof(int32_t) * (size_t)(k > 0 ? k : 1));
    sort_item_t *tmp = (sort_item_t *)malloc(sizeof(sort_item_t) * (size_t)(k > 0 ? k : 1));
    if (!h.score || !h.id || !tmp) {
        c->err = 1;
        free(h.score);
        free(h.id);
        free(tmp);
        return;
    }
    for (int64_t qi = q0; qi < q1; qi++) {
        const float *q = c->xq + qi * d;
        h.size = 0;
        int64_t vi = 0;
        double s4[4];
        for (; vi + 4 <= n; vi += 4) {
            dist4(c->metric, q, c->xb + vi * d, d, s4);
            tk_push(&h, s4[0], (int32_t)vi);
            tk_push(&h, s4[1], (int32_t)(vi + 1));
            tk_push(&h, s4[2], (int32_t)(vi + 2));
            tk_push(&h, s4[3], (int32_t)(vi + 3));
        }
        for (; vi < n; vi++) tk_push(&h, dist1(c->metric, q, c->xb + vi * d, d), (int32_t)vi);
        tk_sorted(&h, c->D + qi * k, c->I + qi * k, tmp);
    }
    free(h.score);
    free(h.id);
    free(tmp);
}

/* Returns 0 on success, -1 on invalid arguments (k == 0 with a non-empty
 * index throws a RangeError in the reference: TopK(0).push reads _score[0]),
 * -2 on allocation failure. */
int orc_flat_search(const float *xb, int64_t n, int64_t d, const float *xq, int64_t nq,
                    int64_t k, int metric, float *D, int32_t *I, int nthreads) {
    if (d <= 0 || n < 0 || nq < 0 || k < 0 || (metric != ORC_L2 && metric != ORC_IP)) return -1;
    if (k == 0) return n > 0 && nq > 0 ? -1 : 0;
    search_ctx_t c = {xb, xq, n, d, k, metric, D, I, 0};
    parallel_for(nq, nthreads, search_range, &c);
    return c.err ? -2 : 0;
}

/* ------------------------------------------------------------------------ */
/* IndexFlat.rangeSearch (index_flat.dart:99-137) -> CSR (index.dart:60-85) */
/* ------------------------------------------------------------------------ */
typedef struct {
    int64_t nq;
    int64_t *lims; /* nq + 1 */
    float *D;
    int32_t *I;
} orc_range_t;

typedef struct {
    int64_t cap, len;
    float *D;
    int32_t *I;
} hitbuf_t;

static int hb_push(hitbuf_t *b, float s, int32_t id) {
    if (b->len == b->cap) {
        int64_t nc = b->cap ? b->cap * 2 : 1024;
        float *nd = (float *)realloc(b->D, sizeof(float) * (size_t)nc);
        if (!nd) return -1;
        b->D = nd;
        int32_t *ni = (int32_t *)realloc(b->I, sizeof(int32_t) * (size_t)nc);
        if (!ni) return -1;
        b->I = ni;
        b->cap = nc;
    }
    b->D[b->len] = s;
    b->I[b->len] = id;
    b->len++;
    return 0;
}

typedef struct {
    const float *xb, *xq;
    int64_t n, d;
    double radius;
    int metric;
    int64_t *counts; /* per query */
    hitbuf_t bufs[256];
    int err;
} range_ctx_t;

static void range_range(void *p, int64_t q0, int64_t q1, int tid) {
    range_ctx_t *c = (range_ctx_t *)p;
    hitbuf_t *b = &c->bufs[tid];
    int64_t d = c->d, n = c->n;
    for (int64_t qi = q0; qi < q1; qi++) {
        const float *q = c->xq + qi * d;
        int64_t before = b->len;
        for (int64_t vi = 0; vi < n; vi++) {
            double s = dist1(c->metric, q, c->xb + vi * d, d);
            int keep = c->metric == ORC_L2 ? (s <= c->radius) : (s >= c->radius);
            if (keep && hb_push(b, (float)s, (int32_t)vi)) {
                c->err = 1;
                return;
            }
        }
        c->counts[qi] = b->len - before;
    }
}

void orc_range_free(orc_range_t *r) {
    if (!r) return;
    free(r->lims);
    free(r->D);
    free(r->I);
    free(r);
}

orc_range_t *orc_flat_range_search(const float *xb, int64_t n, int64_t d, const float *xq,
                                   int64_t nq, double radius, int metric, int nthreads) {
    if (d <= 0 || n < 0 || nq < 0 || (metric != ORC_L2 && metric != ORC_IP)) return NULL;
    range_ctx_t *c = (range_ctx_t *)calloc(1, sizeof(range_ctx_t));
    orc_range_t *r = (orc_range_t *)calloc(1, sizeof(orc_range_t));
    if (!c || !r) {
        free(c);
        free(r);
        return NULL;
    }
    c->xb = xb;
    c->xq = xq;
    c->n = n;
    c->d = d;
    c->radius = radius;
    c->metric = metric;
    c->counts = (int64_t *)calloc((size_t)(nq + 1), sizeof(int64_t));
    r->nq = nq;
    r->lims = (int64_t *)calloc((size_t)(nq + 1), sizeof(int64_t));
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    parallel_for(nq, nthreads, range_range, c);
    int64_t total = 0;
    for (int64_t qi = 0; qi < nq; qi++) {
        r->lims[qi] = total;
        total += c->counts[qi];
    }
    r->lims[nq] = total;
    r->D = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    r->I = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    /* thread t handled a contiguous query block, so concatenating the
     * per-thread buffers in thread order is query order. */
    int64_t w = 0;
    for (int t = 0; t < 256; t++) {
        if (c->bufs[t].len) {
            memcpy(r->D + w, c->bufs[t].D, sizeof(float) * (size_t)c->bufs[t].len);
            memcpy(r->I + w, c->bufs[t].I, sizeof(int32_t) * (size_t)c->bufs[t].len);
            w += c->bufs[t].len;
        }
        free(c->bufs[t].D);
        free(c->bufs[t].I);
    }
    int err = c->err;
    free(c->counts);
    free(c);
    if (err) {
        orc_range_free(r);
        return NULL;
    }
    return r;
}

/* ------------------------------------------------------------------------ */
/* Near-duplicate self-join: IndexFlatIP.rangeSearch(all, thr) keeping pairs */
/* other > qi (bin/vector_dedup_demo.dart:115-128).  Only j > i is scanned; */
/* score(i, j) is the same fp64 expression the demo computes for query i.   */
/* Rows [row_begin, row_end) of the triangle are evaluated (a bounded       */
/* subset for timing); pairs come out sorted by (i, j).                      */
/* ------------------------------------------------------------------------ */
typedef struct {
    int64_t npairs;
    int32_t *i, *j;
    float *s;
} orc_pairs_t;

typedef struct {
    int64_t cap, len;
    int32_t *i, *j;
    float *s;
} pairbuf_t;

static int pb_push(pairbuf_t *b, int32_t i, int32_t j, float s) {
    if (b->len == b->cap) {
        int64_t nc = b->cap ? b->cap * 2 : 1024;
        int32_t *ni = (int32_t *)realloc(b->i, sizeof(int32_t) * (size_t)nc);
        if (!ni) return -1;
        b->i = ni;
        int32_t *nj = (int32_t *)realloc(b->j, sizeof(int32_t) * (size_t)nc);
        if (!nj) return -1;
        b->j = nj;
        float *ns = (float *)realloc(b->s, sizeof(float) * (size_t)nc);
        if (!ns) return -1;
        b->s = ns;
        b->cap = nc;
    }
    b->i[b->len] = i;
    b->j[b->len] = j;
    b->s[b->len] = s;
    b->len++;
    return 0;
}

typedef struct {
    const float *x;
    int64_t n, d, row_begin;
    double thr;
    pairbuf_t bufs[256];
    int err;
} join_ctx_t;

static void join_range(void *p, int64_t r0, int64_t r1, int tid) {
    join_ctx_t *c = (join_ctx_t *)p;
    pairbuf_t *b = &c->bufs[tid];
    int64_t d = c->d, n = c->n;
    for (int64_t ii = r0; ii < r1; ii++) {
        int64_t i = c->row_begin + ii;
        const float *q = c->x + i * d;
        for (int64_t j = i + 1; j < n; j++) {
            double s = dist_ip(q, c->x + j * d, d);
            if (s >= c->thr && pb_push(b, (int32_t)i, (int32_t)j, (float)s)) {
                c->err = 1;
                return;
            }
        }
    }
}

void orc_pairs_free(orc_pairs_t *p) {
    if (!p) return;
    free(p->i);
    free(p->j);
    free(p->s);
    free(p);
}

orc_pairs_t *orc_self_join(const float *x, int64_t n, int64_t d, double thr, int64_t row_begin,
                           int64_t row_end, int nthreads) {
    if (d <= 0 || n < 0 || row_begin < 0 || row_end > n || row_begin > row_end) return NULL;
    join_ctx_t *c = (join_ctx_t *)calloc(1, sizeof(join_ctx_t));
    orc_pairs_t *r = (orc_pairs_t *)calloc(1, sizeof(orc_pairs_t));
    if (!c || !r) {
        free(c);
        free(r);
        return NULL;
    }
    c->x = x;
    c->n = n;
    c->d = d;
    c->thr = thr;
    c->row_begin = row_begin;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    parallel_for(row_end - row_begin, nthreads, join_range, c);
    int64_t total = 0;
    for (int t = 0; t < 256; t++) total += c->bufs[t].len;
    r->npairs = total;
    r->i = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    r->j = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total > 0 ? total : 1));
    r->s = (float *)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    int64_t w = 0;
    for (int t = 0; t < 256; t++) {
        pairbuf_t *b = &c->bufs[t];
        if (b->len) {
            memcpy(r->i + w, b->i, sizeof(int32_t) * (size_t)b->len);
            memcpy(r->j + w, b->j, sizeof(int32_t) * (size_t)b->len);
            memcpy(r->s + w, b->s, sizeof(float) * (size_t)b->len);
            w += b->len;
        }
        free(b->i);
        free(b->j);
        free(b->s);
    }
    int err = c->err;
    free(c);
    if (err) {
        orc_pairs_free(r);
        return NULL;
    }
    return r;
}

/* ------------------------------------------------------------------------ */
/* Kmeans assignment step (kmeans.dart:91-105)                               */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *x, *cen;
    int64_t d, K;
    int32_t *assign;
    double *best;
} assign_ctx_t;

static void assign_range(void *p, int64_t i0, int64_t i1, int tid) {
    (void)tid;
    assign_ctx_t *c = (assign_ctx_t *)p;
    int64_t d = c->d, K = c->K;
    for (int64_t i = i0; i < i1; i++) {
        const float *xi = c->x + i * d;
        int32_t best = 0;
        double best_sq = dist_l2(xi, c->cen, d);
        int64_t cc = 1;
        double s4[4];
        for (; cc + 4 <= K; cc += 4) {
            dist4(ORC_L2, xi, c->cen + cc * d, d, s4);
            for (int u = 0; u < 4; u++) {
                if (s4[u] < best_sq) {
                    best_sq = s4[u];
                    best = (int32_t)(cc + u);
                }
            }
        }
        for (; cc < K; cc++) {
            double ds = dist_l2(xi, c->cen + cc * d, d);
            if (ds < best_sq) {
                best_sq = ds;
                best = (int32_t)cc;
            }
        }
        c->assign[i] = best;
        c->best[i] = best_sq;
    }
}

/* best_sq (optional, n doubles) receives each point's fp64 squared distance
 * to its centroid; *obj is their sum in point order (kmeans.dart:104). */
int orc_kmeans_assign(const float *x, int64_t n, int64_t d, const float *cen, int64_t K,
                      int32_t *assign, double *best_sq, double *obj, int nthreads) {
    if (d <= 0 || n < 0 || K <= 0) return -1;
    double *best = best_sq ? best_sq : (double *)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    if (!best) return -2;
    assign_ctx_t c = {x, cen, d, K, assign, best};
    parallel_for(n, nthreads, assign_range, &c);
    double o = 0.0;
    for (int64_t i = 0; i < n; i++) o += best[i];
    if (obj) *obj = o;
    if (!best_sq) free(best);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Kmeans update step (kmeans.dart:107-140), in place on cen (K x d).        */
/* Empty clusters (count < min_points) copy the currently largest cluster    */
/* (first index among equal counts) plus (u - 0.5) * 1e-4 jitter per         */
/* element; the reference draws u from dart:math Random, here the caller     */
/* passes the u values (njitter doubles in [0,1)), consumed in order.        */
/* Returns the number of jitter values consumed, or -1 if they ran out.      */
/* ------------------------------------------------------------------------ */
int64_t orc_kmeans_update(const float *x, int64_t n, int64_t d, const int32_t *assign, int64_t K,
                          int64_t min_points, float *cen, int32_t *counts, const double *jitter_u,
                          int64_t njitter) {
    float *sums = (float *)calloc((size_t)(K * d), sizeof(float));
    if (!sums) return -2;
    for (int64_t c = 0; c < K; c++) counts[c] = 0;
    for (int64_t i = 0; i < n; i++) {
        int32_t a = assign[i];
        counts[a]++;
        const float *row = x + i * d;
        float *s = sums + (int64_t)a * d;
        /* s[j] += row[j] on a Float32List: exact fp64 sum rounded to fp32,
         * i.e. one correctly rounded fp32 addition */
        for (int64_t j = 0; j < d; j++) s[j] = (float)((double)s[j] + (double)row[j]);
    }
    int64_t used = 0;
    for (int64_t c = 0; c < K; c++) {
        if (counts[c] >= min_points) {
            double inv = 1.0 / (double)counts[c];
            for (int64_t j = 0; j < d; j++) cen[c * d + j] = (float)((double)sums[c * d + j] * inv);
        } else {
            int64_t big = 0;
            for (int64_t cc = 1; cc < K; cc++)
                if (counts[cc] > counts[big]) big = cc;
            for (int64_t j = 0; j < d; j++) {
                if (used >= njitter) {
                    free(sums);
                    return -1;
                }
                double jit = (jitter_u[used++] - 0.5) * 1e-4;
                cen[c * d + j] = (float)((double)cen[big * d + j] + jit);
            }
        }
    }
    free(sums);
    return used;
}
