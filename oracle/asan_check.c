/*
 * asan_check.c -- memory-safety run of the CPU oracle (test infrastructure).
 *
 * Built with AddressSanitizer and UndefinedBehaviorSanitizer by `make -C
 * oracle asan` and run by tests/test_oracle.py.  It includes oracle.c and
 * calls every entry point on shapes that reach the edge paths: ragged d
 * (the scalar tails of the 4-row distance blocks), row and query counts that
 * are not multiples of 4, k above the row count, empty inputs, range results
 * that grow their hit buffers, self-join row windows, and empty k-means
 * clusters.  Any out-of-bounds access or undefined operation aborts with the
 * sanitizer's report; the checks below catch gross mistakes in the results.
 */
#include "oracle.c"

#include <stdio.h>

static uint64_t st = 0x9e3779b97f4a7c15ull;
static double urand(void) {
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    return (double)(st >> 11) * (1.0 / 9007199254740992.0);
}

static float *rows(int64_t n, int64_t d) {
    float *x = (float *)malloc(sizeof(float) * (size_t)(n * d > 0 ? n * d : 1));
    for (int64_t i = 0; i < n * d; i++) x[i] = (float)(urand() * 2.0 - 1.0);
    return x;
}

#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__);  \
            return 1;                                                         \
        }                                                                     \
    } while (0)

int main(void) {
    const int64_t ds[] = {1, 3, 5, 17, 64};
    const int64_t ns[] = {0, 1, 6, 33};
    for (size_t a = 0; a < sizeof ds / sizeof ds[0]; a++)
        for (size_t b = 0; b < sizeof ns / sizeof ns[0]; b++) {
            const int64_t d = ds[a], n = ns[b], nq = 5, k = 7;
            float *xb = rows(n, d), *xq = rows(nq, d);
            float *D = (float *)malloc(sizeof(float) * nq * k);
            int32_t *I = (int32_t *)malloc(sizeof(int32_t) * nq * k);
            for (int metric = 0; metric < 2; metric++)
                for (int nt = 1; nt <= 3; nt += 2) {
                    CHECK(orc_flat_search(xb, n, d, xq, nq, k, metric, D, I, nt) == 0);
                    for (int64_t q = 0; q < nq; q++)
                        for (int64_t j = 0; j < k; j++)
                            CHECK(j < n ? (I[q * k + j] >= 0 && I[q * k + j] < n)
                                        : I[q * k + j] == -1);
                    /* a radius that keeps about half of the hits */
                    orc_range_t *r =
                        orc_flat_range_search(xb, n, d, xq, nq, metric == 0 ? (double)d : 0.0, metric, nt);
                    CHECK(r != NULL && r->lims[0] == 0);
                    for (int64_t q = 0; q < nq; q++) CHECK(r->lims[q + 1] >= r->lims[q]);
                    CHECK(r->lims[nq] <= nq * n);
                    orc_range_free(r);
                }
            /* every row as a query: the range grows past any initial buffer */
            if (n > 0) {
                orc_range_t *r = orc_flat_range_search(xb, n, d, xb, n, 1e30, 0, 2);
                CHECK(r != NULL && r->lims[n] == n * n);
                orc_range_free(r);
                orc_pairs_t *p = orc_self_join(xb, n, d, -1e30, 0, n, 2);
                CHECK(p != NULL && p->npairs == n * (n - 1) / 2);
                orc_pairs_free(p);
                p = orc_self_join(xb, n, d, 0.0, n / 2, n, 3);
                CHECK(p != NULL);
                orc_pairs_free(p);
            }
            /* k-means with more centroids than points: empty clusters take
             * the jitter path */
            if (n > 0) {
                const int64_t K = n + 2;
                float *cen = rows(K, d);
                int32_t *as = (int32_t *)malloc(sizeof(int32_t) * n);
                int32_t *cnt = (int32_t *)malloc(sizeof(int32_t) * K);
                double obj = 0.0, *best = (double *)malloc(sizeof(double) * n);
                double *u = (double *)malloc(sizeof(double) * K * d);
                for (int64_t i = 0; i < K * d; i++) u[i] = urand();
                CHECK(orc_kmeans_assign(xb, n, d, cen, K, as, best, &obj, 2) == 0);
                for (int64_t i = 0; i < n; i++) CHECK(as[i] >= 0 && as[i] < K);
                CHECK(orc_kmeans_update(xb, n, d, as, K, 1, cen, cnt, u, K * d) >= 0);
                free(cen);
                free(as);
                free(cnt);
                free(best);
                free(u);
            }
            CHECK(orc_flat_search(xb, n, d, xq, nq, 0, 0, D, I, 1) == (n > 0 ? -1 : 0));
            free(xb);
            free(xq);
            free(D);
            free(I);
        }
    printf("asan_check ok\n");
    return 0;
}
