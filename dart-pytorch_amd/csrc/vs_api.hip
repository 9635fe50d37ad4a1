// vs_api.hip -- the extern "C" ABI of libvs_hip.so (declared in
// include/vs_hip.h): index lifecycle, planning, host<->device staging,
// error reporting.  All device work of a handle runs on its own stream.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "../../include/vs_hip.h"
#include "vs_internal.h"

namespace {

// (a fixed buffer: reporting an error allocates nothing)
thread_local char g_err[512];

int set_err(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_err(hipError_t e, const char *what) {
    // a failed runtime call (e.g. hipMalloc) also leaves its code as the
    // thread's last error, which the next launch check would read back as
    // its own: clear it once it is reported
    (void)hipGetLastError();
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return set_err(VS_ERR_OOM, "%s: out of device memory (%s)", what, hipGetErrorString(e));
    return set_err(VS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define VS_HIP(call, what)                            \
    do {                                              \
        hipError_t e_ = (call);                       \
        if (e_ != hipSuccess) return hip_err(e_, what); \
    } while (0)

// Restores the caller's current device on scope exit.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Test support (option "fail_alloc"): when > 0, the device or pinned host
// allocation that brings it to 0 fails as out of memory, so tests reach the
// failure paths of every caller (and show that a path allocates nothing).
// Per thread, like the error text.
thread_local int64_t g_fail_alloc = 0;

// Every device allocation of an index goes through here.
hipError_t dev_malloc(void **p, size_t bytes) {
    if (g_fail_alloc > 0 && --g_fail_alloc == 0) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}

// Every pinned host allocation of an index goes through here.
hipError_t host_malloc(void **p, size_t bytes) {
    if (g_fail_alloc > 0 && --g_fail_alloc == 0) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipHostMalloc(p, bytes, hipHostMallocDefault);
}

// Device buffer that only grows.
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need) {
        if (need <= bytes) return hipSuccess;
        if (p) {
            hipError_t e = hipFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            bytes = 0;
        }
        size_t nb = std::max(need, (size_t)4096);
        hipError_t e = dev_malloc(&p, nb);
        if (e != hipSuccess) {
            p = nullptr;
            return e;
        }
        bytes = nb;
        return hipSuccess;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <typename T>
    T *as() const {
        return (T *)p;
    }
};

// Pinned host memory (grown on demand): device-to-host copies into it run
// asynchronously at full link speed.
struct HostBuf {
    void *p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need) {
        if (need <= bytes) return hipSuccess;
        if (p) {
            hipError_t e = hipHostFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            bytes = 0;
        }
        size_t nb = std::max(need, (size_t)4096);
        hipError_t e = host_malloc(&p, nb);
        if (e != hipSuccess) {
            p = nullptr;
            return e;
        }
        bytes = nb;
        return hipSuccess;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <typename T>
    T *as() const {
        return (T *)p;
    }
};

struct ProfEntry {
    int64_t launches = 0;
    double total_ms = 0.0;
};

struct PendingEvent {
    std::string family;
    hipEvent_t a, b;
};

int64_t next_pow2(int64_t v) {
    int64_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

}  // namespace

// Per-handle planner options (vs_index_set_option).  The defaults are the
// tuned plan; the others force a path or a shape so that tests can reach
// every kernel variant on small inputs.
struct VsOptions {
    int gemm = -1;         // GEMM-tiled scan: -1 planner rule (rows >= 256 elements), 0 off, 1 any d
    int gemm_min_nq = 0;   // smallest batch on the GEMM-tiled scan (0: 512 by rule, 256 when forced)
    int gemm_wq = 0, gemm_qb = 0, gemm_kc = 0;  // force a GEMM shape field (0: any)
    int gemm4 = 0;         // GEMM-tiled scan: 1 = the four-wave pipelined kernel where it applies
    int share = -1;        // row-shared scan: -1 rule (rows of 128 elements), 0 off, 1 also 256
    int coarse = 1;        // one-pass bf16 selection of fp32 rows (range, self-join, k-means)
    int copy16 = 1;        // the one-pass selection reads a bf16 copy of the fp32 rows
    int guess = 1;         // large batches: estimated thresholds from a row sample
    int prepass = 1;       // small batches: threshold seeding pre-pass
    int prepass_log2 = 16; // the pre-pass sample: at least 2^prepass_log2 rows
    int scan_kkw = 0;      // >0: per-list keep forced down to this (tests of the verification)
    int scan_nw8 = 0;      // streaming scan: eight waves per workgroup where it fits
    int km16 = 1;          // k-means: the scan reads a bf16 copy of the centroids
    int km16_rt = 4;       // k-means on that copy: 16-row blocks per tile (2 or 4)
    int km16_nqb = 4;      // k-means on that copy: 16-point blocks per wave (2, or 4 with
                           // 32-row tiles)
    int pick_order = 1;    // k-means: the pick walks points grouped by the last step's clusters
    int merge_mu = 0;      // merge: 1024-entry chunks per workgroup pass (0: by batch size; 1, 2,
                           // 4 or 8)
    int merge_g = 0;       // merge: workgroups per query (0: by batch size; 1: one; 2..64: split)
    int guess_div_log2 = 0;  // large batches: the estimate's sample is 1/2^this of the rows (0: 5)
    int kmin_init = 1;       // k-means: start the assign scan's running minima from the last step
    int assign_order = 1;    // k-means: the assign scan walks the points grouped by the last
                             // step's clusters
};

struct vs_index {
    int device = 0;
    VsOptions opt;
    int64_t d = 0;
    int metric = 0;
    int mode = VS_STORAGE_F32;  // requested
    int storage = 0;            // current: 0 fp32, 1 bf16
    int64_t ld = 0;
    int64_t ntotal = 0, cap = 0;
    uint64_t version = 0;  // bumped whenever the stored rows change
    void *xb = nullptr;
    float *xn = nullptr;
    hipStream_t st = nullptr;
    int num_cu = 256;
    size_t lds_max = 64 * 1024;
    // scratch (grown on demand, reused across calls)
    DevBuf stage, qp, qf, qnorm, flags, cand_v, cand_i, lcnt, gthr, lbound, vf, fbq, fbD, fbI, outD, outI,
        athr, rq, ri, rs, rkeep, rcount, misc;
    DevBuf km_cen16, km_c16n;  // k-means: bf16 copy of the centroid rows (and its unused norms)
    DevBuf km_cen, km_cxn, km_assign, km_best, km_fb, km_keys, km_order, km_tmp, km_counts,
        km_offsets, km_out, km_iota;
    // k-means: the points prepared as queries, kept while the rows are unchanged
    DevBuf km_qp, km_qf, km_qnorm;
    // k-means: pinned copies of the distances, assignments and new centroids
    HostBuf km_hbest, km_hassign, km_hcen, km_hfb;
    HostBuf rstage;  // reconstruct: pinned staging of stored rows
    hipStream_t st_copy = nullptr;  // k-means: reads results back beside the update
    // k-means: km_order holds the last step's points grouped by cluster, for
    // these rows (version) and this many points
    uint64_t km_order_version = ~0ull;
    int64_t km_order_n = 0;
    // k-means: km_assign / km_best / km_cen hold a whole step's assignments,
    // squared distances and centroids for these rows (version), points and K
    // (the next step's scan starts its running minima from them)
    DevBuf km_shift, km_init, km_pkeys, km_part;
    uint64_t km_prev_version = ~0ull;
    int64_t km_prev_n = 0, km_prev_K = 0;
    vs::PreparedQueries km_pq;
    uint32_t km_pflags = 0;
    uint64_t km_prep_version = ~0ull;
    // bf16 copy of fp32 rows for the GEMM-tiled one-pass selection (range,
    // self-join), kept while the rows are unchanged
    DevBuf xb16, xb16n;
    uint64_t xb16_version = ~0ull;
    int64_t km_iota_n = -1;  // km_iota holds 0 .. km_iota_n - 1
    bool prof_on = false;
    bool prof_fixed = false;  // inside an allocation-free call: no profiling bookkeeping
    std::map<std::string, ProfEntry> prof;
    // largest stored row norm, for the version of the rows it was taken at
    float xmax_cache = 0.f;
    uint64_t xmax_version = ~0ull;
    DevBuf vx, ctl;  // top-k: exact-path query list, control words
    std::vector<PendingEvent> pending;
};

namespace {

int64_t elem_size(int storage) { return storage == 1 ? 2 : 4; }

int64_t row_bytes(const vs_index *x) { return x->ld * elem_size(x->storage); }

// Brackets a launch with events on the handle's stream when profiling is on.
struct ProfScope {
    vs_index *x;
    const char *fam;
    hipEvent_t a = nullptr, b = nullptr;
    ProfScope(vs_index *x_, const char *fam_) : x(x_), fam(fam_) {
        if (!x->prof_on || x->prof_fixed) return;
        if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
            a = b = nullptr;
            return;
        }
        (void)hipEventRecord(a, x->st);
    }
    ~ProfScope() {
        if (!a) return;
        (void)hipEventRecord(b, x->st);
        x->pending.push_back({fam, a, b});
    }
};

// Counts which scan variant a launch used (always on; read back through
// vs_prof_get with the families "shared", "gemm", "streamed" and
// "streamed8", and per GEMM shape).
void note_scan_kind(vs_index *x, const vs::ScanPlan &plan) {
    x->prof[plan.kind == 3 ? "shared" : plan.kind == 2 ? "gemm" : "streamed"]
        .launches++;
    if (plan.kind == 0 && plan.lw == 8) x->prof["streamed8"].launches++;
    if (plan.kind == 2) {  // and per GEMM shape: "gemm:1,1,2,4,4,2,32"
        char key[64];
        snprintf(key, sizeof key, "gemm:%d,%d,%d,%d,%d,%d,%d", plan.tile_st, plan.tile_pb,
                 plan.lw, plan.g_wq, plan.tile_rb, plan.g_qb, plan.tile_kc);
        x->prof[key].launches++;
    }
}

void prof_collect(vs_index *x) {
    if (x->pending.empty()) return;
    (void)hipStreamSynchronize(x->st);
    for (auto &p : x->pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto &e = x->prof[p.family];
            e.launches++;
            e.total_ms += ms;
        }
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    x->pending.clear();
}

int check_index(const vs_index *x) {
    if (!x) return set_err(VS_ERR_INVALID, "null index handle");
    return VS_OK;
}

// Grows device storage to hold `need` rows; rows past ntotal stay zero and
// kRowSlack slack rows follow the capacity so whole-tile reads of the
// last rows stay inside the allocation.
int ensure_capacity(vs_index *x, int64_t need) {
    if (need <= x->cap) return VS_OK;
    int64_t nc = std::max<int64_t>(need, x->cap * 2);
    nc = std::max<int64_t>(nc, 1024);
    nc = round_up(nc, kRowCapAlign);
    const int64_t rb = row_bytes(x);
    void *nxb = nullptr;
    float *nxn = nullptr;
    const size_t xbytes = (size_t)(nc + kRowSlack) * rb;
    const size_t nbytes = (size_t)(nc + kRowSlack) * sizeof(float);
    VS_HIP(dev_malloc(&nxb, xbytes), "allocating vector storage");
    if (dev_malloc((void **)&nxn, nbytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(nxb);
        return set_err(VS_ERR_OOM, "allocating norm storage (%zu bytes)", nbytes);
    }
    VS_HIP(hipMemsetAsync(nxb, 0, xbytes, x->st), "clearing storage");
    VS_HIP(hipMemsetAsync(nxn, 0, nbytes, x->st), "clearing norms");
    if (x->ntotal > 0) {
        VS_HIP(hipMemcpyAsync(nxb, x->xb, (size_t)x->ntotal * rb, hipMemcpyDeviceToDevice, x->st),
               "copying storage");
        VS_HIP(hipMemcpyAsync(nxn, x->xn, (size_t)x->ntotal * sizeof(float),
                              hipMemcpyDeviceToDevice, x->st),
               "copying norms");
    }
    VS_HIP(hipStreamSynchronize(x->st), "growing storage");
    if (x->xb) (void)hipFree(x->xb);
    if (x->xn) (void)hipFree(x->xn);
    x->xb = nxb;
    x->xn = nxn;
    x->cap = nc;
    return VS_OK;
}

// Validation of n rows already on the device: returns flags.
int device_flags(vs_index *x, const void *src, int dtype, int64_t stride, int64_t n, uint32_t *out) {
    VS_HIP(x->flags.ensure(sizeof(uint32_t)), "flags buffer");
    VS_HIP(hipMemsetAsync(x->flags.p, 0, sizeof(uint32_t), x->st), "clearing flags");
    // store_rows with a throw-away destination computes the flags: use the
    // misc buffer sized for one chunk of rows.
    const int64_t chunk = 1 << 16;
    for (int64_t r = 0; r < n; r += chunk) {
        const int64_t m = std::min(chunk, n - r);
        const int64_t dst_ld = vs::storage_ld(x->d, 0);
        VS_HIP(x->misc.ensure((size_t)m * dst_ld * 4 + (size_t)m * 4), "validation scratch");
        const char *s = (const char *)src + (size_t)r * stride * (dtype == 1 ? 2 : 4);
        VS_HIP(vs::launch_store_rows(s, dtype, stride, m, x->d, x->misc.p, 0, dst_ld,
                                     (float *)((char *)x->misc.p + (size_t)m * dst_ld * 4),
                                     x->flags.as<uint32_t>(), x->st),
               "validating rows");
    }
    VS_HIP(hipMemcpyAsync(out, x->flags.p, sizeof(uint32_t), hipMemcpyDeviceToHost, x->st),
           "reading flags");
    VS_HIP(hipStreamSynchronize(x->st), "validating rows");
    return VS_OK;
}

// Switch bf16 storage to fp32 (AUTO storage meeting a non-bf16 value).
int widen_storage(vs_index *x) {
    const int64_t new_ld = vs::storage_ld(x->d, 0);
    const int64_t nc = std::max<int64_t>(x->cap, 1024);
    void *nxb = nullptr;
    float *nxn = nullptr;
    const size_t xbytes = (size_t)(nc + kRowSlack) * new_ld * 4;
    const size_t nbytes = (size_t)(nc + kRowSlack) * sizeof(float);
    VS_HIP(dev_malloc(&nxb, xbytes), "allocating fp32 storage");
    if (dev_malloc((void **)&nxn, nbytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(nxb);
        return set_err(VS_ERR_OOM, "allocating norm storage");
    }
    VS_HIP(hipMemsetAsync(nxb, 0, xbytes, x->st), "clearing storage");
    VS_HIP(hipMemsetAsync(nxn, 0, nbytes, x->st), "clearing norms");
    VS_HIP(x->flags.ensure(sizeof(uint32_t)), "flags buffer");
    if (x->ntotal > 0)
        VS_HIP(vs::launch_store_rows(x->xb, 1, x->ld, x->ntotal, x->d, nxb, 0, new_ld, nxn,
                                     x->flags.as<uint32_t>(), x->st),
               "widening storage");
    VS_HIP(hipStreamSynchronize(x->st), "widening storage");
    if (x->xb) (void)hipFree(x->xb);
    if (x->xn) (void)hipFree(x->xn);
    x->xb = nxb;
    x->xn = nxn;
    x->cap = nc;
    x->ld = new_ld;
    x->storage = 0;
    ++x->version;
    return VS_OK;
}

int add_device_rows(vs_index *x, const void *src, int dtype, int64_t n) {
    uint32_t f = 0;
    int rc = device_flags(x, src, dtype, x->d, n, &f);
    if (rc) return rc;
    if (f & vs::kFlagNonFinite)
        return set_err(VS_ERR_NONFINITE, "vectors contain NaN or infinity");
    if (x->mode == VS_STORAGE_AUTO && x->storage == 1 && (f & vs::kFlagNotBf16)) {
        rc = widen_storage(x);
        if (rc) return rc;
    }
    rc = ensure_capacity(x, x->ntotal + n);
    if (rc) return rc;
    VS_HIP(x->flags.ensure(sizeof(uint32_t)), "flags buffer");
    char *dst = (char *)x->xb + (size_t)x->ntotal * row_bytes(x);
    VS_HIP(vs::launch_store_rows(src, dtype, x->d, n, x->d, dst, x->storage, x->ld,
                                 x->xn + x->ntotal, x->flags.as<uint32_t>(), x->st),
           "storing rows");
    VS_HIP(hipStreamSynchronize(x->st), "storing rows");
    x->ntotal += n;
    ++x->version;
    return VS_OK;
}

int check_dtype(int dt) {
    if (dt != VS_DTYPE_F32 && dt != VS_DTYPE_BF16)
        return set_err(VS_ERR_INVALID, "dtype must be VS_DTYPE_F32 or VS_DTYPE_BF16 (got %d)", dt);
    return VS_OK;
}

// ---------------------------------------------------------------------------
// Planning
// ---------------------------------------------------------------------------
// GEMM-tiled planning (large batches): the first built shape for this
// storage and query-plane count whose LDS fits, then the number of database
// splits so that the grid fills whole rounds of workgroups.  Each query has
// one candidate list per row wave (lw) in a workgroup, so a list keeps at
// least kk_final / lw entries and the block's lists together bound the
// query's kk_final-th value.  The grid targets two rounds of workgroups per
// CU; query blocks go in groups of 32 per XCD.  The options gemm,
// gemm_min_nq and gemm_wq / gemm_qb / gemm_kc force it on or off and pick a
// shape.

// The row-shared scan's lists.  Top-k lists (lane): one per lane, four per
// query and workgroup (each lane sees rows 4g .. 4g + 3 of every 16-row
// block), each keeping kk (kk_final, or kk_final / 4 with the merge's
// verification); a lane's list gains up to 4 entries per row block and is
// cut before a tile when it holds more than cap - 4 rt, and cap leaves kk +
// 4 rt slots above kk so that cuts stay rare.  Otherwise (k-means lists,
// estimates) one list per query and workgroup keeping kk_final, cut when it
// holds more than cap - 16 rt; 256 slots at least keep cuts rare while its
// threshold is still loose (the list is sorted only up to its fill).
bool share_lists(const vs_index *x, vs::ScanPlan *p, bool lane) {
    const int rt = p->tm;
    const int kk = lane ? p->kk : p->kk_final;
    const int cap = lane ? (int)std::max<int64_t>(64, next_pow2(2 * kk + 4 * rt))
                         : (int)std::max<int64_t>(256, next_pow2(kk + std::max(48, 16 * rt)));
    const size_t lds = vs::share_lds_bytes(p->nks, p->bn / 64, rt, cap, lane ? 4 : 1);
    if (lds > x->lds_max) return false;
    p->kk = kk;
    p->cap = cap;
    p->lw = lane ? 4 : 1;
    p->lds_bytes = lds;
    return true;
}

// Row-shared scan (top-k only): bf16 rows of 128 or 256 elements, one query
// plane, large batches.  Option share: -1 = planner rule (rows of 128
// elements, batch >= 256), 0 = off, 1 = also rows of 256 elements.  The
// one-pass selection of fp32 rows (storage kSelectCoarse, k-means) takes
// rows of 128 and 256 elements.  The grid is four times the resident
// workgroups.  lane: top-k lane lists (bf16 rows by default); false for
// the estimate pre-pass (lists of each lane's smallest values, one per query).
bool plan_share(const vs_index *x, int64_t nq, int64_t nrows, int planes, int storage,
                vs::ScanPlan *p, int64_t max_split, int lane = -1) {
    const int mode = x->opt.share;
    if (mode == 0 || (storage != 1 && storage != vs::kSelectCoarse) || planes != 1) return false;
    if (!(x->ld == 128 || (x->ld == 256 && (mode > 0 || storage == vs::kSelectCoarse))))
        return false;
    if (nq < 256) return false;
    const int nks = (int)(x->ld / 32), nqb = nks == 4 ? 4 : 2;
    // fp32 tiles: half the rows, the same staging registers
    const int rt = storage == 1 ? (nks == 4 ? 8 : 4) : 2;
    vs::ScanPlan sp = *p;
    sp.nks = nks;
    sp.bn = 64 * nqb;
    sp.tm = rt;
    // bf16 rows: top-k lists; the one-pass selection: k-means lists
    if (!share_lists(x, &sp, lane < 0 ? storage == 1 : lane > 0)) return false;
    *p = sp;
    p->kind = 3;
    p->tile_st = storage;
    p->share_topm = 0;
    const size_t lds = p->lds_bytes;
    p->nqblk = (nq + p->bn - 1) / p->bn;
    const int64_t tile_rows = 16 * rt;
    // Splits: the whole grid resident at once (or whole rounds of it), so the
    // query blocks of a split -- dealt to one XCD back to back -- walk its
    // rows together through that XCD's L2, and no round is left half empty.
    const int bpc = std::max(1, vs::share_blocks_per_cu(storage, nks, p->bn, rt, x->ld, lds, 0));
    const int64_t resident = (int64_t)std::max(1, x->num_cu) * bpc;
    const int64_t target = resident * 4;
    int64_t nsplit = std::max<int64_t>(1, target / p->nqblk);
    nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, nrows / (tile_rows * 8)));
    if (max_split > 0) nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, max_split / p->lw));
    int64_t rps = round_up((nrows + nsplit - 1) / nsplit, tile_rows);
    if (rps <= 0) rps = tile_rows;
    p->rows_per_split = rps;
    p->nsplit = std::max<int64_t>(1, (nrows + rps - 1) / rps);
    return true;
}

bool plan_gemm(const vs_index *x, int64_t nq, int64_t nrows, int planes, int storage,
               bool kk_forced, vs::ScanPlan *p) {
    // default: large batches of long rows (measured on MI355X: the GEMM-tiled
    // scan beats the streaming one at d = 768, batch >= 1024, and on the
    // k-means assign at d = 256; at d = 128 the streaming scan's 20 waves per
    // CU hide its list work better)
    const VsOptions &o = x->opt;
    const int mode = o.gemm;
    if (mode == 0) return false;
    if (mode < 0 && x->ld < 256) return false;
    if (nq < (o.gemm_min_nq > 0 ? o.gemm_min_nq : mode < 0 ? 512 : 256)) return false;
    struct Shape {
        int st, pb, wr, wq, rb, qb, kc;
    };
#define VS_GSHAPE_ENTRY(ST_, PB_, WR_, WQ_, RB_, QB_, KC_) {ST_, PB_, WR_, WQ_, RB_, QB_, KC_},
    static const Shape shapes[] = {VS_GEMM_SHAPES(VS_GSHAPE_ENTRY)};
#undef VS_GSHAPE_ENTRY
    const int fwq = o.gemm_wq, fqb = o.gemm_qb, fkc = o.gemm_kc;
    const Shape *pick = nullptr;
    int kk = p->kk, cap = 0;
    size_t lds = 0;
    // the four-wave pipelined kernel: bf16 rows whose stride is whole
    // groups of four 32-element K-chunks, one query plane
    static const Shape pipe4 = {1, 1, 2, 2, 4, 4, 32};
    p->g_pipe = 0;
    if (o.gemm4 && storage == 1 && planes == 1 && x->ld % 128 == 0 && (!fwq || fwq == 2) &&
        (!fqb || fqb == 4) && (!fkc || fkc == 32)) {
        kk = p->kk;
        if (!kk_forced && kk < p->kk_final) kk = std::max(kk, p->kk_final / pipe4.wr);
        cap = (int)next_pow2(kk + 32 * pipe4.rb + 16);
        lds = vs::gemm4_lds_bytes(cap);
        if (lds <= x->lds_max) {
            pick = &pipe4;
            p->g_pipe = 1;
        }
    }
    for (const Shape &sh : shapes) {
        if (pick) break;
        if (sh.st != storage || sh.pb != planes) continue;
        if (fwq && sh.wq != fwq) continue;
        if (fqb && sh.qb != fqb) continue;
        if (fkc && sh.kc != fkc) continue;
        if (x->ld % sh.kc) continue;
        kk = p->kk;
        if (!kk_forced && kk < p->kk_final) kk = std::max(kk, p->kk_final / sh.wr);
        // a wave may append up to 32 * rb entries per query and row tile
        cap = (int)next_pow2(kk + 32 * sh.rb + 16);
        lds = vs::gemm_lds_bytes(sh.st, sh.pb, sh.wr, sh.wq, sh.rb, sh.qb, sh.kc, cap);
        if (lds > x->lds_max) continue;
        pick = &sh;
        break;
    }
    if (!pick) return false;
    p->kind = 2;
    p->kk = kk;
    p->cap = cap;
    p->bn = 32 * pick->wq * pick->qb;
    p->lw = pick->wr;
    p->g_wq = pick->wq;
    p->g_qb = pick->qb;
    p->tile_rb = pick->rb;
    p->tile_kc = pick->kc;
    p->tile_st = pick->st;
    p->tile_pb = pick->pb;
    p->nks = 0;
    p->lds_bytes = lds;
    p->nqblk = (nq + p->bn - 1) / p->bn;
    // query blocks per XCD group: the most (up to 32, a power of two) whose
    // query planes take <= 1.5 MiB, so that they stay in the XCD's 4 MiB L2
    // beside the rows; a chunk of the grid (group x split run, about one
    // XCD's resident workgroups) covers 32 / group splits
    const int64_t qbytes = (int64_t)p->bn * x->ld * 2 * planes;
    int64_t qg = 1;
    while (qg < 32 && 2 * qg * qbytes <= (int64_t)3 << 19) qg *= 2;
    p->tile_group = std::max<int64_t>(1, std::min<int64_t>(p->nqblk, qg));
    int64_t spc = std::max<int64_t>(1, 32 / p->tile_group);
    const int64_t tile_rows = (int64_t)pick->wr * 32 * pick->rb;
    const int64_t ncu = (int64_t)std::max(1, x->num_cu);
    int64_t max_split = std::max<int64_t>(1, nrows / (tile_rows * 4));
    // a short scan that would leave CUs idle (a pre-pass over a small
    // sample) takes splits down to one tile each
    if (p->nqblk * max_split < ncu)
        max_split = std::max<int64_t>(
            max_split, std::min<int64_t>((nrows + tile_rows - 1) / tile_rows,
                                         (ncu + p->nqblk - 1) / p->nqblk));
    const int64_t rounds = 2;
    // smallest split count whose grid covers the target rounds of CUs and
    // fills >= 90% of its last round; else the best fill seen
    int64_t best = 1;
    double best_score = -1.0;
    for (int64_t ns = 1; ns <= max_split; ++ns) {
        const int64_t blocks = p->nqblk * ns;
        const double eff = (double)blocks / (double)(((blocks + ncu - 1) / ncu) * ncu);
        if (blocks >= rounds * ncu && eff >= 0.9) {
            best = ns;
            break;
        }
        const double score = std::min(1.0, (double)blocks / (double)(rounds * ncu)) * eff;
        if (score > best_score) {
            best_score = score;
            best = ns;
        }
        if (blocks >= 4 * rounds * ncu) break;
    }
    // at least one split run per group (its workgroups then walk different
    // splits together instead of idling the XCD)
    best = std::max(best, std::min(spc, max_split));
    int64_t rps = round_up((nrows + best - 1) / best, tile_rows);
    if (rps <= 0) rps = tile_rows;
    p->rows_per_split = rps;
    p->nsplit = std::max<int64_t>(1, (nrows + rps - 1) / rps);
    p->tile_spc = std::min(spc, p->nsplit);
    return true;
}

// Scan planning.  kk_final candidates per query survive the merge; each
// wave's list keeps kk of them: kk_final itself up to 32, else kk_final / 4
// (then four lists of a block together bound the kk_final-th value, and the
// merge verifies that no list dropped a winner; safe forces kk = kk_final;
// the option scan_kkw forces a shorter keep, for tests of the verification
// path).  The streaming scan targets four workgroups per CU.
// min_tiles: the fewest row tiles a split of the streaming scan gets (its
// lists warm up over them; the threshold-seeding scans over small samples
// use fewer, so that their short sample still spreads over every CU)
// list_budget > 0: the candidate lists may take at most this many bytes
// (streaming scan only; its split count shrinks to fit).
int plan_scan_core(const vs_index *x, int64_t nq, int64_t nrows, int planes, int64_t kk_final,
                   int storage, vs::ScanPlan *p, bool safe, int64_t max_lists, bool range,
                   int min_tiles, size_t list_budget) {
    int64_t kk = kk_final <= 32 ? kk_final : kk_final / 4;
    const int kkw = x->opt.scan_kkw;
    if (kkw > 0) kk = std::min<int64_t>(kk_final, std::max<int64_t>(4, next_pow2(kkw)));
    if (safe) kk = kk_final;
    p->kk_final = (int)kk_final;
    p->kk = (int)kk;
    p->cap = (int)next_pow2(kk + 48);
    // 16-row blocks per wave tile: one for short rows (d <= 128: measured
    // faster on 1M x 128, the epilogue dominates), two otherwise
    p->tm = x->ld <= 128 && storage == 1 ? 1 : 2;
    p->kind = 0;
    if (!range && kkw <= 0 && !list_budget &&
        plan_share(x, nq, nrows, planes, storage, p, max_lists))
        return VS_OK;
    // (a list limit shapes the split count of the row-shared and streaming
    // scans; the GEMM-tiled scan makes few lists per query anyway)
    if (!list_budget && plan_gemm(x, nq, nrows, planes, storage, kkw > 0 || safe, p)) return VS_OK;
    const int nks = (int)(x->ld / 32);
    const int cands[3] = {64, 32, 16};
    p->bn = 0;
    p->nks = 0;
    for (int bn : cands) {
        if (bn > 16 && round_up(nq, 16) < bn) continue;
        const bool qreg = storage == 1 && planes == 1 && (nks == 4 || nks == 8) &&
                          nks * (bn / 16) <= 16;
        if (vs::scan_lds_bytes(bn, qreg ? 0 : planes, x->ld, p->cap, 4) <= x->lds_max) {
            p->bn = bn;
            p->nks = qreg ? nks : 0;
            break;
        }
    }
    if (!p->bn)
        return set_err(VS_ERR_UNSUPPORTED,
                       "d=%lld is too large for the LDS-resident query block of this build",
                       (long long)x->d);
    // eight waves per workgroup when the LDS-resident query block leaves room
    // for a single workgroup per CU (bf16 rows): twice the loads in flight
    // (option scan_nw8: measured slightly slower than four waves on
    // 20M x 768 bf16, so off by default)
    p->lw = 4;
    if (storage == 1 && !p->nks && p->tm == 2 && x->opt.scan_nw8 &&
        2 * vs::scan_lds_bytes(p->bn, planes, x->ld, p->cap, 4) > x->lds_max &&
        vs::scan_lds_bytes(p->bn, planes, x->ld, p->cap, 8) <= x->lds_max)
        p->lw = 8;
    p->lds_bytes = vs::scan_lds_bytes(p->bn, p->nks ? 0 : planes, x->ld, p->cap, p->lw);
    p->nqblk = (nq + p->bn - 1) / p->bn;
    const int64_t tile_rows = 16 * p->lw * p->tm;  // rows per block per round
    const int64_t target = (int64_t)x->num_cu * 4;
    int64_t nsplit = std::max<int64_t>(1, (target + p->nqblk - 1) / p->nqblk);
    const int64_t min_rows = tile_rows * std::max(1, min_tiles);
    int64_t by_rows = (nrows + min_rows - 1) / min_rows;
    // a short scan that would leave most CUs idle takes splits down to one
    // tile each (up to one workgroup per CU): each wave then works alone on
    // its SIMD and its time is mostly memory latency, so more splits, not
    // warmer lists, shorten it
    if (p->nqblk * by_rows < x->num_cu)
        by_rows = std::max<int64_t>(
            by_rows, std::min<int64_t>((nrows + tile_rows - 1) / tile_rows,
                                       std::max<int64_t>(1, x->num_cu / p->nqblk)));
    nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, by_rows));
    if (max_lists > 0) nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, max_lists / p->lw));
    if (list_budget > 0) {
        const size_t per_split = (size_t)p->nqblk * p->lw * p->bn * p->cap * 8;
        nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, (int64_t)(list_budget / per_split)));
    }
    int64_t rps = round_up((nrows + nsplit - 1) / nsplit, tile_rows);
    if (rps <= 0) rps = tile_rows;
    p->rows_per_split = rps;
    p->nsplit = std::max<int64_t>(1, (nrows + rps - 1) / rps);
    return VS_OK;
}

// The merge's shape.  One workgroup per query reads the query's lists in
// passes of merge_mu 1024-entry chunks: a batch that leaves most CUs idle
// reads more chunks per pass (more loads in flight per workgroup), and, when
// a quarter of the workgroups that fit on the CUs at once would still
// outnumber the queries, splits each query's entries over merge_g workgroups
// (all resident at once, >= 1024 entries each, at most 64) whose kk_final
// best pairs a second pass merges.  Called again when the lists' kind
// changes (uncut lists hold more entries).
void plan_merge(const vs_index *x, int64_t nq, vs::ScanPlan *p) {
    int mu = x->opt.merge_mu;
    if (!mu) mu = nq <= x->num_cu ? 8 : nq <= 4 * x->num_cu ? 4 : 1;
    while (mu > 1 && vs::merge_lds_bytes(x->ld, mu) > x->lds_max) mu >>= 1;
    p->merge_mu = mu;
    int64_t g = x->opt.merge_g;
    if (!g) {
        const bool counted = p->kind == 3 || (p->kind == 0 && p->uncut);
        const int64_t entries = p->nsplit * p->lw * (counted ? p->cap : p->kk);
        const int64_t per_cu = std::max<int64_t>(
            1, (int64_t)(x->lds_max / std::max<size_t>(1, vs::merge_lds_bytes(x->ld, mu))));
        g = (int64_t)x->num_cu * per_cu / std::max<int64_t>(1, nq);
        g = g < 4 ? 1 : std::min<int64_t>({g, 64, entries / 1024});
    }
    p->merge_g = (int)std::max<int64_t>(1, g);
}

int plan_scan(const vs_index *x, int64_t nq, int64_t nrows, int planes, int64_t kk_final,
              int storage, vs::ScanPlan *p, bool safe = false, int64_t max_lists = 0,
              bool range = false, int min_tiles = 8, size_t list_budget = 0) {
    const int rc = plan_scan_core(x, nq, nrows, planes, kk_final, storage, p, safe, max_lists,
                                  range, min_tiles, list_budget);
    if (rc == VS_OK) plan_merge(x, nq, p);
    return rc;
}

// Device scratch of one call.  Ordinary calls use the index's grow-on-demand
// buffers, plus call-local ones for the fallback paths; the allocation-free
// entry point carves every piece, in order, from one fixed device region
// (mark / reset release what a finished sub-step carved).
struct Arena {
    char *base = nullptr;  // fixed region, or null
    size_t cap = 0, used = 0;
    std::vector<DevBuf> local;  // ordinary calls: call-local buffers
    Arena() = default;
    Arena(const Arena &) = delete;
    Arena &operator=(const Arena &) = delete;
    ~Arena() {
        for (auto &b : local) b.release();
    }
    bool fixed() const { return base != nullptr; }
    int carve(size_t bytes, void **p, const char *what) {
        const size_t off = (used + 255) & ~(size_t)255;
        if (off + bytes > cap)
            return set_err(VS_ERR_UNSUPPORTED,
                           "%s: %zu bytes past the end of the %zu-byte fixed scratch", what,
                           off + bytes - cap, cap);
        *p = base + off;
        used = off + bytes;
        return VS_OK;
    }
    // the index's buffer b with at least `bytes` (a fresh piece when fixed)
    int get(DevBuf &b, size_t bytes, void **p, const char *what) {
        if (base) return carve(bytes, p, what);
        VS_HIP(b.ensure(bytes), what);
        *p = b.p;
        return VS_OK;
    }
    // a buffer of this call only
    int tmp(size_t bytes, void **p, const char *what) {
        if (base) return carve(bytes, p, what);
        local.emplace_back();
        VS_HIP(local.back().ensure(bytes), what);
        *p = local.back().p;
        return VS_OK;
    }
    size_t mark() const { return used; }
    void reset(size_t m) { used = m; }
};

#define VS_TAKE(arena_call)          \
    do {                             \
        int rc_ = (arena_call);      \
        if (rc_) return rc_;         \
    } while (0)

// Rows of prepared queries (and of the per-query shared thresholds): a
// multiple of 256 plus 256 spare rows, so the query blocks of any scan plan
// -- nqblk * bn <= nq + bn - 1 with bn <= 256, and bn need not divide 256 --
// lie inside the buffers.  scan_fits() checks every plan against it.
int64_t query_pad(int64_t nq) { return round_up(std::max<int64_t>(nq, 1), 256) + 256; }

int scan_fits(const vs::ScanPlan &plan, const vs::PreparedQueries &pq) {
    if (plan.bn > 256 || plan.nqblk * plan.bn > pq.nq_pad)
        return set_err(VS_ERR_UNSUPPORTED,
                       "internal: scan plan covers %lld query rows, only %lld are prepared",
                       (long long)(plan.nqblk * plan.bn), (long long)pq.nq_pad);
    return VS_OK;
}

// Builds the MFMA query planes, the fp32 copy and the norms of nq query rows
// (device memory, `stride` elements apart); *flags_out receives the query
// flags (non-finite, not bf16).  The planes and copies go to qp / qf / qnorm
// (the index's buffers) or, in a fixed arena, to fresh pieces of it.
// defer_flags (a zeroed device word) for bf16 queries: their plane count is
// one whatever the values, so the flags go to that word, to be read with the
// results, and nothing waits here (a row with a non-finite value is prepared
// as the unit vector e_0, so that the search runs on finite values).  With
// spec_one_plane, fp32 queries take the same path with one plane on trust
// (both planes are written): the caller reads the flags with its results and
// searches again with two planes if any query was not bf16-exact.
int prepare_queries(vs_index *x, Arena &A, const void *q_dev, int q_dtype, int64_t stride,
                    int64_t nq, vs::PreparedQueries *pq, uint32_t *flags_out, DevBuf &qp,
                    DevBuf &qf, DevBuf &qnorm, uint32_t *defer_flags = nullptr,
                    bool spec_one_plane = false) {
    pq->nq = nq;
    pq->nq_pad = query_pad(nq);
    void *p_qp, *p_qf, *p_qn, *p_fl;
    VS_TAKE(A.get(qp, (size_t)pq->nq_pad * 2 * x->ld * 2, &p_qp, "query planes"));
    VS_TAKE(A.get(qf, (size_t)std::max<int64_t>(nq, 1) * x->d * 4, &p_qf, "query copy"));
    VS_TAKE(A.get(qnorm, (size_t)pq->nq_pad * 4, &p_qn, "query norms"));
    pq->qp = (uint16_t *)p_qp;
    pq->qf = (float *)p_qf;
    pq->qnorm = (float *)p_qn;
    if (defer_flags && (q_dtype == VS_DTYPE_BF16 || spec_one_plane)) {
        VS_HIP(vs::launch_prepare_queries(q_dev, q_dtype, stride, nq, x->d, x->ld, x->metric, *pq,
                                          defer_flags, x->st),
               "preparing queries");
        pq->planes = 1;
        if (flags_out) *flags_out = 0;
        return VS_OK;
    }
    VS_TAKE(A.get(x->flags, sizeof(uint32_t), &p_fl, "flags buffer"));
    VS_HIP(vs::launch_fill32(p_fl, 1, 0u, x->st), "clearing flags");
    VS_HIP(vs::launch_prepare_queries(q_dev, q_dtype, stride, nq, x->d, x->ld, x->metric, *pq,
                                      (uint32_t *)p_fl, x->st),
           "preparing queries");
    uint32_t f = 0;
    VS_HIP(hipMemcpyAsync(&f, p_fl, sizeof f, hipMemcpyDeviceToHost, x->st), "query flags");
    VS_HIP(hipStreamSynchronize(x->st), "preparing queries");
    if (f & vs::kFlagNonFinite) return set_err(VS_ERR_NONFINITE, "queries contain NaN or infinity");
    pq->planes = (f & vs::kFlagNotBf16) ? 2 : 1;
    if (flags_out) *flags_out = f;
    return VS_OK;
}

int prepare_queries(vs_index *x, Arena &A, const void *q_dev, int q_dtype, int64_t stride,
                    int64_t nq, vs::PreparedQueries *pq, uint32_t *flags_out,
                    uint32_t *defer_flags = nullptr, bool spec_one_plane = false) {
    return prepare_queries(x, A, q_dev, q_dtype, stride, nq, pq, flags_out, x->qp, x->qf,
                           x->qnorm, defer_flags, spec_one_plane);
}

__global__ void fill_sentinels_kernel(float *D, int32_t *I, int64_t m, float v) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < m) {
        D[t] = v;
        I[t] = -1;
    }
}

// Candidate lists of a scan and of its threshold pre-passes (which run
// first and reuse the same memory): values, ids, and per-list counts with
// the largest count after them.
struct ListBufs {
    float *v = nullptr;
    int32_t *i = nullptr;
    int32_t *cnt = nullptr;
    size_t elems = 0, lists = 0;
};

size_t list_count(const vs::ScanPlan &p) { return (size_t)p.nqblk * p.nsplit * p.lw * p.bn; }
// the lists, then the split merge's partial area
size_t list_elems(const vs::ScanPlan &p) {
    const size_t part = p.merge_g > 1 ? (size_t)p.nqblk * p.bn * p.merge_g * p.kk_final : 0;
    return list_count(p) * p.cap + part;
}

int take_lists(vs_index *x, Arena &A, size_t elems, size_t lists, ListBufs *L) {
    void *pv, *pi, *pc;
    VS_TAKE(A.get(x->cand_v, elems * 4, &pv, "candidate lists"));
    VS_TAKE(A.get(x->cand_i, elems * 4, &pi, "candidate lists"));
    VS_TAKE(A.get(x->lcnt, (lists + 1) * 4, &pc, "list counts"));
    L->v = (float *)pv;
    L->i = (int32_t *)pi;
    L->cnt = (int32_t *)pc;
    L->elems = elems;
    L->lists = lists;
    return VS_OK;
}

// A plan warms up badly when it makes many lists per query over many rows.
// Rows per sampled row of the small-batch threshold pre-pass.
constexpr int kPrepassDiv = 1024;

bool needs_seed(const vs_index *x, const vs::ScanPlan &plan) {
    return plan.kind == 0 && plan.nsplit * plan.lw >= 512 && x->ntotal >= (1 << 18);
}

// Seeds every query's shared threshold (gthr) from the first S rows: a scan
// of those rows with the ordinary plan -- itself seeded from the first S / 32
// rows when that plan would warm up badly too -- and a merge that sets the
// threshold one code above the kk_final-th smallest accumulator value of the
// query's lists.  kk_final rows of the full scan lie strictly below it, so
// the full scan loses nothing; thresholds only ever tighten.  The candidate
// lists are scratch here (the full scan rewrites them).
//
// seed_rank > 0 makes the threshold an estimate instead of a bound: one code
// above the seed_rank-th smallest value of the sample, which the caller
// chooses so that the full scan very likely holds kk_final rows below it;
// the merge then flags the queries for which it does not (guess_thresholds).
//
// L == nullptr plans only: *need_elems / *need_lists grow to what the
// pre-pass scans need.
int seed_thresholds(vs_index *x, const vs::PreparedQueries &pq, int64_t S, int64_t kk_final,
                    uint32_t *gthr, ListBufs *L, size_t *need_elems, size_t *need_lists,
                    int seed_rank = 0, int64_t max_lists = -1, size_t list_budget = 0) {
    S = std::min<int64_t>(S, x->ntotal);
    vs::ScanPlan pp;
    if (max_lists < 0) max_lists = 0;
    int rc = plan_scan(x, pq.nq, S, pq.planes, kk_final, x->storage, &pp, false, max_lists, false,
                       2, list_budget);
    if (rc) return rc;
    // an estimate needs only the values of the sample's seed_rank smallest:
    // the row-shared scan then keeps each lane's smallest in registers
    // instead of lists (exact unless one lane met more than m of them; then
    // the estimate is larger, never smaller)
    if (pp.kind == 3 && seed_rank > 0 && seed_rank <= 4 * vs::share_topm_est()) {
        vs::ScanPlan tp = pp;
        if (plan_share(x, pq.nq, S, pq.planes, x->storage, &tp, max_lists, 0)) {
            pp = tp;
            pp.share_topm = vs::share_topm_est();
            plan_merge(x, pq.nq, &pp);
        }
    }
    // the streaming scan's lists over a short sample end full: the merge
    // reads them uncut (cutting each list at the end costs more than the
    // merge's extra reads), and an entry a list dropped in a cut lies above
    // that list's kk-th value, so the merged rank-r value can only be larger
    // (still a bound, or a larger estimate)
    if (pp.kind == 0) {
        pp.uncut = 1;
        plan_merge(x, pq.nq, &pp);
    }
    if ((rc = scan_fits(pp, pq))) return rc;
    const int div = kPrepassDiv;
    if (pp.kind == 0 && pp.nsplit * pp.lw >= 512 && S >= (1 << 18)) {
        rc = seed_thresholds(x, pq, std::max<int64_t>((int64_t)1 << x->opt.prepass_log2, S / div),
                             kk_final, gthr, L,
                             need_elems, need_lists, 0, -1, list_budget);
        if (rc) return rc;
    }
    // the GEMM-tiled estimate pre-pass: its lists would warm up on their own
    // share of the sample (most of its tiles then take the append path); a
    // bound on the kk_final-th value of the first 1/32 of the sample lets it
    // start tight (the sample's own kk_final smallest all lie below it, so
    // the estimate is unchanged)
    if (pp.kind == 2 && seed_rank > 0 && S >= (1 << 16)) {
        rc = seed_thresholds(x, pq, S / 32, kk_final, gthr, L, need_elems, need_lists, 0, -1,
                             list_budget);
        if (rc) return rc;
    }
    if (!L) {
        *need_elems = std::max(*need_elems, list_elems(pp));
        *need_lists = std::max(*need_lists, list_count(pp));
        return VS_OK;
    }
    if (list_elems(pp) > L->elems || list_count(pp) > L->lists)
        return set_err(VS_ERR_HIP, "internal: pre-pass lists larger than planned");
    const bool prof = !x->prof_fixed;
    VS_HIP(vs::launch_fill32(L->cnt + list_count(pp), 1, 0u, x->st), "list counts");
    {
        ProfScope ps(x, "prepass");
        VS_HIP(vs::launch_scan_topk(x->xb, x->storage, x->ld, x->xn, S, x->metric, pq, pp, L->v,
                                    L->i, gthr, nullptr, L->cnt, x->st),
               "seeding scan");
    }
    VS_HIP(vs::launch_merge_threshold(pq, pp, L->v, L->i, gthr, x->ld, seed_rank, L->cnt, x->st),
           "seeding threshold");
    if (prof) x->prof["prepass_scans"].launches++;
    if (prof && pp.merge_g > 1 && !(seed_rank > 0 && seed_rank <= 64))
        x->prof["split_merges"].launches++;
    return VS_OK;
}

// Large batches: every list of the full scan warms up on its own share of
// the rows, and their thresholds stay far above the query's final
// kk_final-th value for most of the scan.  An estimate taken from a sample
// is much tighter: with S of the N rows scanned first, the j-th smallest
// sample value has on average j * N / S rows of the full scan below it, and
// fewer than kk_final only when kk_final rows would hold j sample rows,
// about P(Poisson(kk_final * S / N) >= j) for rows in random order.  j is
// chosen four standard deviations and four rows above that mean (below 1e-5
// per query for every kk_final this build allows).  Queries whose estimate
// was too tight are found by the merge and searched again exactly.
bool needs_guess(const vs_index *x, const vs::ScanPlan &plan, int64_t nq) {
    return x->opt.guess && nq >= 256 &&
           x->ntotal >= (1 << 18) && plan.nsplit * plan.lw * plan.kk >= 4 * plan.kk_final;
}

// The sample is 1/2^div_log2 of the rows (option guess_div_log2, 1/32 by
// default): a smaller one costs less to scan but leaves more candidates to
// the full scan (about j 2^div_log2 rows per query lie below the estimate).
// Measured on 20M x 768 bf16 at batch 1024 and 8192 (GEMM-tiled scan): 1/64
// to 1/256 cut the pre-pass from 2.0 / 12.8 ms to 0.6-1.2 / 2.5-7.4 ms but
// slowed the full scan by 2-5 %, about the same per step; 1/32 keeps the
// full scan fastest.
int guess_div_log2(const vs_index *x) {
    return x->opt.guess_div_log2 ? x->opt.guess_div_log2 : 5;
}

int guess_thresholds(vs_index *x, const vs::PreparedQueries &pq, int64_t kk_final, int div_log2,
                     uint32_t *gthr, ListBufs *L, size_t *need_elems, size_t *need_lists) {
    const int64_t S =
        std::min<int64_t>(x->ntotal, std::max<int64_t>(4096, x->ntotal >> div_log2));
    const double lam = (double)kk_final * (double)S / (double)x->ntotal;
    const int j = (int)std::ceil(lam + 4.0 * std::sqrt(lam) + 4.0);
    const int64_t kkp = std::max<int64_t>(8, next_pow2(j));
    if (L && !x->prof_fixed) x->prof["guess_scans"].launches++;
    return seed_thresholds(x, pq, S, kkp, gthr, L, need_elems, need_lists, j, 12);
}

// The largest stored row norm (times 1 + 1e-6), cached per row version.
int xnorm_max(vs_index *x, Arena &A, float *out) {
    if (x->ntotal == 0) {
        *out = 0.f;
        return VS_OK;
    }
    if (x->xmax_version != x->version) {
        void *p;
        VS_TAKE(A.get(x->misc, sizeof(float), &p, "norm maximum"));
        VS_HIP(vs::launch_max_reduce(x->xn, x->ntotal, (float *)p, x->st), "norm maximum");
        float m = 0.f;
        VS_HIP(hipMemcpyAsync(&m, p, sizeof m, hipMemcpyDeviceToHost, x->st), "norm maximum");
        VS_HIP(hipStreamSynchronize(x->st), "norm maximum");
        x->xmax_cache = std::sqrt(m) * (1.0f + 1e-6f);
        x->xmax_version = x->version;
    }
    *out = x->xmax_cache;
    return VS_OK;
}

// Accumulator error model of a top-k scan of these rows with these queries
// (relative error of one product of MFMA operands; the accumulation factor
// covers up to three passes of d products and the fp32 row norms):
//   bf16 rows, queries exactly bf16 (one plane): products exact;
//   bf16 rows, two query planes: the dropped residual, below 2^-18;
//   fp32 rows (hi + lo planes), one query plane: below 2^-18;
//   fp32 rows, two query planes: lo * q1 and the residuals, below 3.1 * 2^-18.
// The factors below are 2.7 to 4 times those.
// fp32 accumulation of npass MFMA passes over d elements (bf16 rows: one
// pass per query plane; fp32 rows: hi x plane 0, lo x plane 0 [, hi x plane
// 1]): at most npass d + 1 terms, each rounding at most one unit of a
// truncating fp32 accumulator, 2^-23 (round-to-nearest would be 2^-24);
// tests/test_gpu_mfma_rounding.py holds both MFMA shapes to this on
// adversarial operands.
double accum_gamma(int64_t d, int npass) {
    return ((double)npass * (double)d + 4.0) * (1.0 / 8388608.0);
}

void topk_error_model(const vs_index *x, int planes, vs::TopkCheck *chk) {
    chk->err_g = (float)accum_gamma(x->d, x->storage == 1 ? planes : 1 + planes);
    if (x->storage == 1)
        chk->err_r = planes == 1 ? 0.f : (float)(1.0 / 65536.0);
    else
        chk->err_r = planes == 1 ? (float)(1.0 / 65536.0) : (float)(1.0 / 32768.0);
}

int search_device(vs_index *x, Arena &A, const void *q_dev, int q_dtype, int64_t nq, int64_t k,
                  float *D, int32_t *I, bool safe = false, size_t list_budget = 0);

// Exact top-k of nq fp32 query rows (device, [nq][d]) without the MFMA
// selection: per-(query, split) lists of the kk best exact keys, then the
// merge (k <= kMaxFusedK), or a per-query sort of every row's key (larger
// k; not in a fixed arena).
int exact_search(vs_index *x, Arena &A, const float *qf, int64_t nq, int64_t k, float *D,
                 int32_t *I) {
    if (nq <= 0) return VS_OK;
    const int64_t kk = std::max<int64_t>(8, next_pow2(k + std::max<int64_t>(4, k / 4)));
    if (kk <= 512) {
        // splits: a few workgroups per CU over all queries, >= 1024 rows each
        const int64_t target = (int64_t)x->num_cu * 4;
        int64_t ns = std::max<int64_t>(1, (target + nq - 1) / nq);
        ns = std::min<int64_t>(ns, std::max<int64_t>(1, x->ntotal / 1024));
        if (A.fixed())  // the lists stay within 16 MiB
            ns = std::max<int64_t>(1, std::min<int64_t>(ns, (int64_t)(16 << 20) / (nq * kk * 8)));
        const int64_t rps = round_up((x->ntotal + ns - 1) / ns, 256);
        ns = (x->ntotal + rps - 1) / rps;
        void *pv, *pi;
        VS_TAKE(A.tmp((size_t)nq * ns * kk * 4, &pv, "exact lists"));
        VS_TAKE(A.tmp((size_t)nq * ns * kk * 4, &pi, "exact lists"));
        VS_HIP(vs::launch_exact_lists(x->xb, x->storage, x->ld, x->d, x->metric, qf, nq, x->ntotal,
                                      (int)kk, ns, rps, (float *)pv, (int32_t *)pi, x->st),
               "exact lists");
        vs::PreparedQueries pq;
        pq.qf = (float *)qf;
        pq.nq = nq;
        pq.nq_pad = nq;
        vs::ScanPlan plan;
        plan.kind = 0;
        plan.bn = 1;
        plan.lw = 1;
        plan.kk = (int)kk;
        plan.kk_final = (int)kk;
        plan.cap = (int)kk;
        plan.nqblk = nq;
        plan.nsplit = ns;
        void *pf;
        VS_TAKE(A.get(x->flags, sizeof(uint32_t), &pf, "flags buffer"));
        VS_HIP(vs::launch_fill32(pf, 1, 0u, x->st), "clearing flags");
        VS_HIP(vs::launch_merge_refine(x->xb, x->storage, x->ld, x->d, x->metric, pq, plan,
                                       (float *)pv, (int32_t *)pi, nullptr, nullptr, nullptr,
                                       nullptr, k, D, I, x->ntotal, (uint32_t *)pf, 0, nullptr,
                                       nullptr, x->st),
               "exact merge");
        if (!x->prof_fixed) x->prof["exact_queries"].launches += nq;
        return VS_OK;
    }
    if (A.fixed())
        return set_err(VS_ERR_UNSUPPORTED, "k=%lld needs the sorting path, which allocates",
                       (long long)k);
    // one query chunk of keys within 1 GiB, plus the sort's output and scratch
    const int64_t n = x->ntotal;
    const int64_t qchunk = std::max<int64_t>(1, std::min<int64_t>(nq, (int64_t)(1 << 27) / n));
    size_t tmp_bytes = 0;
    VS_HIP(vs::exact_sort_topk(x->xb, x->storage, x->ld, x->d, x->metric, qf, nq, n, k, D, I,
                               nullptr, qchunk, nullptr, tmp_bytes, x->st),
           "sort size");
    void *keys, *tmp;
    VS_TAKE(A.tmp((size_t)(qchunk + 1) * n * 8, &keys, "sort keys"));
    VS_TAKE(A.tmp(tmp_bytes + 256, &tmp, "sort scratch"));
    VS_HIP(vs::exact_sort_topk(x->xb, x->storage, x->ld, x->d, x->metric, qf, nq, n, k, D, I,
                               (uint64_t *)keys, qchunk, tmp, tmp_bytes, x->st),
           "exact sort");
    if (!x->prof_fixed) x->prof["exact_sort_queries"].launches += nq;
    return VS_OK;
}

// Re-search of the queries listed in list_dev (device, m entries) of the
// prepared queries pq: their rows are gathered, searched by `how` (0: the
// MFMA selection again with full-length lists and no estimates; 1: the
// exact path), and their k results scattered back into D / I.
int research_listed(vs_index *x, Arena &A, const vs::PreparedQueries &pq, const int32_t *list_dev,
                    int64_t m, int64_t k, float *D, int32_t *I, int how) {
    if (m <= 0) return VS_OK;
    void *lst, *fq, *fD, *fI;
    VS_TAKE(A.tmp((size_t)m * 4, &lst, "fallback list"));
    VS_TAKE(A.tmp((size_t)m * x->d * 4, &fq, "fallback queries"));
    VS_TAKE(A.tmp((size_t)m * k * 4, &fD, "fallback results"));
    VS_TAKE(A.tmp((size_t)m * k * 4, &fI, "fallback results"));
    VS_HIP(hipMemcpyAsync(lst, list_dev, (size_t)m * 4, hipMemcpyDeviceToDevice, x->st),
           "fallback list");
    VS_HIP(vs::launch_gather_rows(pq.qf, (const int32_t *)lst, m, x->d, fq, x->st),
           "fallback gather");
    const size_t mk = A.mark();
    int rc = how == 0 ? search_device(x, A, fq, VS_DTYPE_F32, m, k, (float *)fD, (int32_t *)fI,
                                      true, A.fixed() ? (size_t)(48 << 20) : 0)
                      : exact_search(x, A, (const float *)fq, m, k, (float *)fD, (int32_t *)fI);
    if (rc) return rc;
    VS_HIP(vs::launch_scatter_rows(fD, (const int32_t *)lst, m, k, D, x->st), "fallback scatter");
    VS_HIP(vs::launch_scatter_rows(fI, (const int32_t *)lst, m, k, I, x->st), "fallback scatter");
    A.reset(mk);
    if (!x->prof_fixed) x->prof[how == 0 ? "fallback" : "exact_fallback"].launches += m;
    return VS_OK;
}

// Top-k search of nq device query rows into device D / I [nq][k].  safe:
// full-length lists and no threshold estimates (the re-search of queries
// the merge could not prove exact).  list_budget > 0 bounds the bytes of
// the candidate lists (the streaming scan's split count adapts).
int search_device(vs_index *x, Arena &A, const void *q_dev, int q_dtype, int64_t nq, int64_t k,
                  float *D, int32_t *I, bool safe, size_t list_budget) {
    if (nq < 0 || k < 0) return set_err(VS_ERR_INVALID, "nq and k must be >= 0");
    if (nq == 0) return VS_OK;
    if (k == 0) {
        if (x->ntotal == 0) return VS_OK;
        // TopK(0).push reads _score[0] of an empty list (index.dart:248-260)
        return set_err(VS_ERR_INVALID, "k must be >= 1 for a non-empty index");
    }
    if (x->ntotal == 0) {
        const int64_t m = nq * k;
        fill_sentinels_kernel<<<dim3((unsigned)((m + 255) / 256)), dim3(256), 0, x->st>>>(
            D, I, m, x->metric == 0 ? __builtin_huge_valf() : -__builtin_huge_valf());
        VS_HIP(hipGetLastError(), "filling sentinels");
        VS_HIP(hipStreamSynchronize(x->st), "search");
        return VS_OK;
    }
    const int64_t kk = std::max<int64_t>(8, next_pow2(k + std::max<int64_t>(4, k / 4)));
    // control words: merge flags, the counts of the two lists, then the
    // query flags of bf16 queries (read with the results)
    void *p_ctl;
    VS_TAKE(A.get(x->ctl, 4 * sizeof(int32_t), &p_ctl, "control words"));
    int32_t *ctl = (int32_t *)p_ctl;
    VS_HIP(vs::launch_fill32(ctl, 4, 0u, x->st), "control words");
    vs::PreparedQueries pq;
    // fp32 queries on bf16 rows: one query plane on trust (nothing waits for
    // the query flags, which are read with the results); the rare batch with
    // a query that bf16 does not hold is searched again with two planes (not
    // in a fixed arena, whose scratch holds one search)
    const bool spec = kk <= 512 && q_dtype != VS_DTYPE_BF16 && x->storage == 1 && !A.fixed();
    int rc = prepare_queries(x, A, q_dev, q_dtype, x->d, nq, &pq, nullptr,
                             kk <= 512 ? (uint32_t *)(ctl + 3) : nullptr, spec);
    if (rc) return rc;
    if (kk > 512) {  // beyond the fused selection: the sorting path
        rc = exact_search(x, A, pq.qf, nq, k, D, I);
        if (rc) return rc;
        VS_HIP(hipStreamSynchronize(x->st), "search");
        return VS_OK;
    }
    for (int attempt = 0;; ++attempt) {
        vs::ScanPlan plan;
        rc = plan_scan(x, nq, x->ntotal, pq.planes, kk, x->storage, &plan, safe, 0, false, 8,
                       list_budget);
        if (rc) return rc;
        if ((rc = scan_fits(plan, pq))) return rc;
        const bool verify = plan.kk < plan.kk_final;
        const bool guess = !safe && needs_guess(x, plan, nq);
        const bool seed = !guess && !safe && needs_seed(x, plan) && x->opt.prepass;
        const int64_t seed_S =
            std::max<int64_t>((int64_t)1 << x->opt.prepass_log2, x->ntotal / kPrepassDiv);
        // candidate lists for the scan and its pre-passes
        size_t elems = list_elems(plan), lists = list_count(plan);
        const int gdl = guess_div_log2(x);
        if (guess) rc = guess_thresholds(x, pq, kk, gdl, nullptr, nullptr, &elems, &lists);
        else if (seed) rc = seed_thresholds(x, pq, seed_S, kk, nullptr, nullptr, &elems, &lists, 0, -1, list_budget);
        if (rc) return rc;
        ListBufs L;
        VS_TAKE(take_lists(x, A, elems, lists, &L));
        void *p_gthr, *p_lb = nullptr, *p_vf, *p_vx;
        VS_TAKE(A.get(x->gthr, (size_t)pq.nq_pad * 4, &p_gthr, "shared thresholds"));
        if (verify) VS_TAKE(A.get(x->lbound, list_count(plan) * 4, &p_lb, "list bounds"));
        VS_TAKE(A.get(x->vf, (size_t)(nq + 1) * 4, &p_vf, "verification list"));
        VS_TAKE(A.get(x->vx, (size_t)(nq + 1) * 4, &p_vx, "exactness list"));
        uint32_t *gthr = (uint32_t *)p_gthr;
        VS_HIP(vs::launch_fill32(gthr, pq.nq_pad, vs::kGthrInit, x->st), "shared thresholds");
        // Small batches over many rows make many short lists, each warming up on
        // its own (every list must fill kk entries before its threshold means
        // anything).  Seeding the shared thresholds from samples first (see
        // seed_thresholds) lets the full scan start tight; large batches start
        // from an estimate (guess_thresholds).
        size_t e0 = 0, l0 = 0;
        if (guess) rc = guess_thresholds(x, pq, kk, gdl, gthr, &L, &e0, &l0);
        else if (seed) rc = seed_thresholds(x, pq, seed_S, kk, gthr, &L, &e0, &l0, 0, -1, list_budget);
        if (rc) return rc;
        if (!x->prof_fixed) note_scan_kind(x, plan);
        VS_HIP(vs::launch_fill32(L.cnt + list_count(plan), 1, 0u, x->st), "list counts");
        {
            ProfScope ps(x, "scan");
            VS_HIP(vs::launch_scan_topk(x->xb, x->storage, x->ld, x->xn, x->ntotal, x->metric, pq, plan,
                                        L.v, L.i, gthr, (float *)p_lb, L.cnt, x->st),
                   "scan kernel");
        }
        vs::TopkCheck chk;
        VS_TAKE(xnorm_max(x, A, &chk.xmax));
        topk_error_model(x, pq.planes, &chk);
        chk.vx_count = ctl + 2;
        chk.vx_list = (int32_t *)p_vx;
        {
            ProfScope ps(x, "merge");
            VS_HIP(vs::launch_merge_refine(x->xb, x->storage, x->ld, x->d, x->metric, pq, plan, L.v, L.i,
                                           gthr, (float *)p_lb, ctl + 1, (int32_t *)p_vf, k, D, I,
                                           x->ntotal, (uint32_t *)ctl, guess ? 1 : 0, L.cnt, &chk,
                                           x->st),
                   "merge kernel");
        }
        if (!x->prof_fixed && plan.merge_g > 1) x->prof["split_merges"].launches++;
        int32_t hc[4] = {0, 0, 0, 0};
        VS_HIP(hipMemcpyAsync(hc, ctl, sizeof hc, hipMemcpyDeviceToHost, x->st), "merge flags");
        VS_HIP(hipStreamSynchronize(x->st), "search");
        if (attempt == 0 && spec && ((uint32_t)hc[3] & vs::kFlagNotBf16) &&
            !((uint32_t)hc[3] & vs::kFlagNonFinite)) {
            pq.planes = 2;  // (both planes were prepared)
            VS_HIP(vs::launch_fill32(ctl, 3, 0u, x->st), "control words");
            continue;
        }
        if ((uint32_t)hc[3] & vs::kFlagNonFinite)
            return set_err(VS_ERR_NONFINITE, "queries contain NaN or infinity");
        if ((uint32_t)hc[0] & vs::kFlagBadId)
            return set_err(VS_ERR_HIP, "internal error: a candidate id outside the index reached the merge");
        // queries whose shortened lists may have dropped a winner, or whose
        // estimated threshold left fewer than kk_final candidates, are searched
        // again with full-length lists and no estimate; queries whose selection
        // the accumulator's error could have changed go to the exact path
        // (both rare for unordered data)
        // (the exact path first: the re-search prepares its queries into the
        // index's query buffers, which both gathers read)
        rc = research_listed(x, A, pq, (const int32_t *)p_vx, hc[2], k, D, I, 1);
        if (rc) return rc;
        rc = research_listed(x, A, pq, (const int32_t *)p_vf, hc[1], k, D, I, 0);
        if (rc) return rc;
        VS_HIP(hipStreamSynchronize(x->st), "search");
        return VS_OK;
    }
}

struct RangeHits {
    std::vector<int32_t> q, id;
    std::vector<float> s;
};

// Candidate scan + exact re-test; hits sorted by (query, id).
int range_core(vs_index *x, const vs::PreparedQueries &pq, double radius, int self_join,
               uint32_t qflags, RangeHits *out) {
    out->q.clear();
    out->id.clear();
    out->s.clear();
    if (pq.nq == 0 || x->ntotal == 0) return VS_OK;
    // one-pass selection of fp32 rows where the GEMM-tiled scan runs it: the
    // acceptance bounds widen to its error and every hit is re-tested exactly
    vs::ScanPlan plan;
    int rc = VS_OK;
    bool coarse = x->storage == 0 && x->opt.coarse;
    if (coarse)
        coarse = plan_scan(x, pq.nq, x->ntotal, 1, 8, vs::kSelectCoarse, &plan, false, 0, true) ==
                     VS_OK &&
                 plan.kind == 2;
    if (!coarse) {
        plan = vs::ScanPlan();
        rc = plan_scan(x, pq.nq, x->ntotal, pq.planes, 8, x->storage, &plan, false, 0, true);
        if (rc) return rc;
    }
    if ((rc = scan_fits(plan, pq))) return rc;
    // the one-pass selection multiplies the rows' bf16 rounding: it reads a
    // bf16 copy of them (half the bytes, no conversion in the kernel) with
    // the fp32 rows' norms, when the copy fits in memory
    const void *scan_rows = x->xb;
    int scan_storage = x->storage;
    if (coarse && plan.tile_st == vs::kSelectCoarse && x->opt.copy16) {
        const size_t bytes = (size_t)(x->ntotal + kRowSlack) * x->ld * 2;
        if (x->xb16_version != x->version) {
            x->xb16_version = ~0ull;
            if (x->xb16.ensure(bytes) == hipSuccess &&
                x->xb16n.ensure((size_t)(x->ntotal + kRowSlack) * 4) == hipSuccess) {
                VS_HIP(hipMemsetAsync(x->xb16.p, 0, bytes, x->st), "row copy");
                VS_HIP(x->flags.ensure(4), "flags");
                VS_HIP(vs::launch_store_rows(x->xb, 0, x->ld, x->ntotal, x->ld, x->xb16.p, 1, x->ld,
                                             x->xb16n.as<float>(), x->flags.as<uint32_t>(), x->st),
                       "row copy");
                x->xb16_version = x->version;
            } else {
                (void)hipGetLastError();
                x->xb16.release();
                x->xb16n.release();
            }
        }
        if (x->xb16_version == x->version) {
            // the copy holds bf16 rows: their own plan (the four-wave
            // pipelined kernel applies to them)
            vs::ScanPlan p16;
            if (plan_scan(x, pq.nq, x->ntotal, 1, 8, 1, &p16, false, 0, true) == VS_OK &&
                p16.kind == 2 && p16.bn <= 256 && p16.nqblk * p16.bn <= pq.nq_pad)
                plan = p16;
            plan.tile_st = 1;
            scan_rows = x->xb16.p;
            scan_storage = 1;
        }
    }
    Arena A;
    float xmax = 0.f;
    VS_TAKE(xnorm_max(x, A, &xmax));
    VS_HIP(x->athr.ensure((size_t)pq.nq * 4), "range bounds");
    const int exact_q = (qflags & vs::kFlagNotBf16) ? 0 : 1;
    const int exact_x = x->storage == 1 ? 1 : 0;
    VS_HIP(vs::launch_range_bounds(pq, x->d, x->metric, radius, xmax, exact_q, exact_x, coarse,
                                   x->athr.as<float>(), x->st),
           "range bounds");
    VS_HIP(x->rcount.ensure(sizeof(unsigned long long)), "range counter");
    int64_t cap = std::max<int64_t>(1 << 20, pq.nq * 4);
    unsigned long long found = 0;
    for (int attempt = 0; attempt < 2; ++attempt) {
        VS_HIP(x->rq.ensure((size_t)cap * 4), "range candidates");
        VS_HIP(x->ri.ensure((size_t)cap * 4), "range candidates");
        VS_HIP(hipMemsetAsync(x->rcount.p, 0, sizeof(unsigned long long), x->st), "range counter");
        note_scan_kind(x, plan);
        {
            ProfScope ps(x, self_join ? "join" : "range");
            VS_HIP(vs::launch_scan_range(scan_rows, scan_storage, x->ld, x->xn, x->ntotal, pq, plan,
                                         x->athr.as<float>(), self_join, x->metric,
                                         x->rq.as<int32_t>(), x->ri.as<int32_t>(),
                                         x->rcount.as<unsigned long long>(), cap, x->st),
                   "range scan");
        }
        VS_HIP(hipMemcpyAsync(&found, x->rcount.p, sizeof found, hipMemcpyDeviceToHost, x->st),
               "range count");
        VS_HIP(hipStreamSynchronize(x->st), "range scan");
        if ((int64_t)found <= cap) break;
        cap = (int64_t)found;  // second pass stores everything
    }
    const int64_t m = (int64_t)found;
    if (m == 0) return VS_OK;
    VS_HIP(x->rs.ensure((size_t)m * 4), "range scores");
    VS_HIP(x->rkeep.ensure((size_t)m), "range flags");
    {
        ProfScope ps(x, "refine");
        VS_HIP(hipMemsetAsync(x->flags.p, 0, sizeof(uint32_t), x->st), "clearing flags");
        VS_HIP(vs::launch_range_refine(x->xb, x->storage, x->ld, x->d, x->metric, pq.qf,
                                       x->rq.as<int32_t>(), x->ri.as<int32_t>(), m, radius,
                                       x->rs.as<float>(), x->rkeep.as<uint8_t>(), x->ntotal, pq.nq,
                                       x->flags.as<uint32_t>(), x->st),
               "range refine");
    }
    std::vector<int32_t> cq(m), ci(m);
    std::vector<float> cs(m);
    std::vector<uint8_t> keep(m);
    VS_HIP(hipMemcpyAsync(cq.data(), x->rq.p, (size_t)m * 4, hipMemcpyDeviceToHost, x->st), "D2H");
    VS_HIP(hipMemcpyAsync(ci.data(), x->ri.p, (size_t)m * 4, hipMemcpyDeviceToHost, x->st), "D2H");
    VS_HIP(hipMemcpyAsync(cs.data(), x->rs.p, (size_t)m * 4, hipMemcpyDeviceToHost, x->st), "D2H");
    VS_HIP(hipMemcpyAsync(keep.data(), x->rkeep.p, (size_t)m, hipMemcpyDeviceToHost, x->st), "D2H");
    uint32_t rflags = 0;
    VS_HIP(hipMemcpyAsync(&rflags, x->flags.p, sizeof rflags, hipMemcpyDeviceToHost, x->st), "D2H");
    VS_HIP(hipStreamSynchronize(x->st), "range results");
    if (rflags & vs::kFlagBadId)
        return set_err(VS_ERR_HIP, "internal error: a range candidate outside the index");
    std::vector<int64_t> idx;
    idx.reserve(m);
    for (int64_t t = 0; t < m; ++t)
        if (keep[t]) idx.push_back(t);
    std::sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) {
        return cq[a] != cq[b] ? cq[a] < cq[b] : ci[a] < ci[b];
    });
    out->q.resize(idx.size());
    out->id.resize(idx.size());
    out->s.resize(idx.size());
    for (size_t t = 0; t < idx.size(); ++t) {
        out->q[t] = cq[idx[t]];
        out->id[t] = ci[idx[t]];
        out->s[t] = cs[idx[t]];
    }
    return VS_OK;
}

}  // namespace

namespace {

// ---------------------------------------------------------------------------
// Fixed scratch of the allocation-free search (vs_index_search_device_noalloc).
// Each device holds its own instance of `scratch` from module load until the
// process ends; host code never passes the array's name to a kernel (it is a
// host-side stand-in), only the device address hipGetSymbolAddress returns,
// taken once per device with that device current.
// ---------------------------------------------------------------------------
constexpr size_t kFixedScratchBytes = (size_t)128 << 20;
constexpr size_t kFixedListBudget = (size_t)32 << 20;  // main scan's candidate lists
constexpr int64_t kFixedMaxNq = 64, kFixedMaxK = 128, kFixedMaxD = 4096;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) char scratch[kFixedScratchBytes];

namespace {

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_call_mu[kMaxDevices];  // serialises the calls that use one device's region

// The device address of this device's scratch (the current device must be
// `device`).
int fixed_scratch(int device, char **out) {
    if (device < 0 || device >= kMaxDevices)
        return set_err(VS_ERR_UNSUPPORTED, "device %d: fixed scratch covers devices 0..%d", device,
                       kMaxDevices - 1);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_err(e, "hipGetSymbolAddress(scratch)");
        if (!p) return set_err(VS_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[device] = p;
    }
    *out = (char *)g_scratch_ptr[device];
    return VS_OK;
}

}  // namespace

// ===========================================================================
// ABI
// ===========================================================================
extern "C" {

const char *vs_last_error(void) { return g_err; }

int vs_device_count(int *count) {
    if (!count) return set_err(VS_ERR_INVALID, "null count");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) {
        *count = 0;
        return set_err(VS_ERR_NO_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(e));
    }
    *count = c;
    return VS_OK;
}

int vs_device_name(int device, char *buf, int64_t len) {
    if (!buf || len <= 0) return set_err(VS_ERR_INVALID, "null or empty name buffer");
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return hip_err(e, "hipGetDeviceProperties");
    // the marketing name can be empty (some drivers leave it blank): the
    // architecture, CU count and memory size name the part then
    snprintf(buf, (size_t)len, "%s (%s, %d CUs, %.0f GiB)", p.name[0] ? p.name : "HIP device",
             p.gcnArchName, p.multiProcessorCount, (double)p.totalGlobalMem / (1024.0 * 1024 * 1024));
    return VS_OK;
}

int vs_index_create(int device, int64_t d, int metric, int storage, vs_index **out) {
    if (!out) return set_err(VS_ERR_INVALID, "null output handle");
    *out = nullptr;
    if (d <= 0) return set_err(VS_ERR_INVALID, "d must be > 0 (got %lld)", (long long)d);
    if (metric != VS_METRIC_L2 && metric != VS_METRIC_IP)
        return set_err(VS_ERR_INVALID, "unknown metric code %d", metric);
    if (storage != VS_STORAGE_F32 && storage != VS_STORAGE_BF16 && storage != VS_STORAGE_AUTO)
        return set_err(VS_ERR_INVALID, "unknown storage code %d", storage);
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return set_err(VS_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count)
        return set_err(VS_ERR_INVALID, "device %d out of range [0, %d)", device, count);
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    vs_index *x = new (std::nothrow) vs_index();
    if (!x) return set_err(VS_ERR_OOM, "host allocation");
    x->device = device;
    x->d = d;
    x->metric = metric;
    x->mode = storage;
    x->storage = storage == VS_STORAGE_F32 ? 0 : 1;
    x->ld = vs::storage_ld(d, x->storage);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) == hipSuccess) {
        x->num_cu = p.multiProcessorCount;
        x->lds_max = p.sharedMemPerBlock;
    }
    hipError_t e = hipStreamCreateWithFlags(&x->st, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete x;
        return hip_err(e, "hipStreamCreate");
    }
    *out = x;
    return VS_OK;
}

void vs_index_destroy(vs_index *x) {
    if (!x) return;
    DeviceGuard g(x->device);
    if (x->st) (void)hipStreamSynchronize(x->st);
    for (auto &p : x->pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    if (x->xb) (void)hipFree(x->xb);
    if (x->xn) (void)hipFree(x->xn);
    DevBuf *bufs[] = {&x->stage,   &x->qp,        &x->qf,       &x->qnorm,    &x->flags, &x->gthr,
                      &x->lbound,  &x->vf,        &x->fbq,      &x->fbD,      &x->fbI,
                      &x->cand_v,  &x->cand_i,    &x->outD,     &x->outI,     &x->athr,
                      &x->rq,      &x->ri,        &x->rs,       &x->rkeep,    &x->rcount,
                      &x->misc,    &x->km_cen,    &x->km_cxn,   &x->km_assign, &x->km_best,
                      &x->km_fb,   &x->km_keys,   &x->km_order, &x->km_tmp,   &x->km_counts,
                      &x->km_offsets, &x->km_out, &x->km_iota, &x->lcnt,   &x->km_qp,
                      &x->km_qf,   &x->km_qnorm,  &x->km_cen16, &x->km_c16n, &x->xb16,
                      &x->xb16n,   &x->vx,        &x->ctl,      &x->km_shift, &x->km_init,
                      &x->km_pkeys, &x->km_part};
    for (DevBuf *b : bufs) b->release();
    x->km_hbest.release();
    x->km_hassign.release();
    x->km_hcen.release();
    x->km_hfb.release();
    x->rstage.release();
    if (x->st_copy) {
        (void)hipStreamSynchronize(x->st_copy);
        (void)hipStreamDestroy(x->st_copy);
    }
    if (x->st) (void)hipStreamDestroy(x->st);
    delete x;
}

int vs_index_reserve(vs_index *x, int64_t n) {
    if (int rc = check_index(x)) return rc;
    if (n < 0) return set_err(VS_ERR_INVALID, "n must be >= 0");
    if (n > (int64_t)INT32_MAX)
        return set_err(VS_ERR_INVALID, "n = %lld rows exceeds the int32 id range", (long long)n);
    DeviceGuard g(x->device);
    return ensure_capacity(x, n);
}

int vs_index_reset(vs_index *x) {
    if (int rc = check_index(x)) return rc;
    DeviceGuard g(x->device);
    if (x->ntotal > 0) {
        VS_HIP(hipMemsetAsync(x->xb, 0, (size_t)x->ntotal * row_bytes(x), x->st), "reset");
        VS_HIP(hipMemsetAsync(x->xn, 0, (size_t)x->ntotal * 4, x->st), "reset");
        VS_HIP(hipStreamSynchronize(x->st), "reset");
    }
    x->ntotal = 0;
    ++x->version;
    return VS_OK;
}

int64_t vs_index_ntotal(const vs_index *x) { return x ? x->ntotal : -1; }
int64_t vs_index_d(const vs_index *x) { return x ? x->d : -1; }
int vs_index_metric(const vs_index *x) { return x ? x->metric : -1; }
int vs_index_storage(const vs_index *x) { return x ? x->storage : -1; }

int vs_index_add(vs_index *x, const void *xs, int src_dtype, int64_t n) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(src_dtype)) return rc;
    if (n < 0) return set_err(VS_ERR_INVALID, "n must be >= 0");
    if (n == 0) return VS_OK;
    if (!xs) return set_err(VS_ERR_INVALID, "null vectors");
    if (x->ntotal + n > (int64_t)INT32_MAX)
        return set_err(VS_ERR_INVALID, "ids are int32: ntotal + n must stay below 2^31");
    DeviceGuard g(x->device);
    const int64_t es = src_dtype == 1 ? 2 : 4;
    const int64_t rowb = x->d * es;
    // validate everything before storing anything (add is all-or-nothing)
    const int64_t chunk = std::max<int64_t>(1, (int64_t)(256 << 20) / rowb);
    bool any_not_bf16 = false;
    for (int64_t r = 0; r < n; r += chunk) {
        const int64_t m = std::min(chunk, n - r);
        VS_HIP(x->stage.ensure((size_t)m * rowb), "staging buffer");
        VS_HIP(hipMemcpyAsync(x->stage.p, (const char *)xs + (size_t)r * rowb, (size_t)m * rowb,
                              hipMemcpyHostToDevice, x->st),
               "uploading vectors");
        uint32_t f = 0;
        int rc = device_flags(x, x->stage.p, src_dtype, x->d, m, &f);
        if (rc) return rc;
        if (f & vs::kFlagNonFinite)
            return set_err(VS_ERR_NONFINITE, "vectors contain NaN or infinity");
        any_not_bf16 |= (f & vs::kFlagNotBf16) != 0;
    }
    if (x->mode == VS_STORAGE_AUTO && x->storage == 1 && any_not_bf16) {
        int rc = widen_storage(x);
        if (rc) return rc;
    }
    int rc = ensure_capacity(x, x->ntotal + n);
    if (rc) return rc;
    VS_HIP(x->flags.ensure(sizeof(uint32_t)), "flags buffer");
    for (int64_t r = 0; r < n; r += chunk) {
        const int64_t m = std::min(chunk, n - r);
        VS_HIP(hipMemcpyAsync(x->stage.p, (const char *)xs + (size_t)r * rowb, (size_t)m * rowb,
                              hipMemcpyHostToDevice, x->st),
               "uploading vectors");
        char *dst = (char *)x->xb + (size_t)(x->ntotal + r) * row_bytes(x);
        VS_HIP(vs::launch_store_rows(x->stage.p, src_dtype, x->d, m, x->d, dst, x->storage, x->ld,
                                     x->xn + x->ntotal + r, x->flags.as<uint32_t>(), x->st),
               "storing rows");
        VS_HIP(hipStreamSynchronize(x->st), "storing rows");
    }
    x->ntotal += n;
    ++x->version;
    return VS_OK;
}

int vs_index_add_device(vs_index *x, const void *xs_dev, int src_dtype, int64_t n) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(src_dtype)) return rc;
    if (n < 0) return set_err(VS_ERR_INVALID, "n must be >= 0");
    if (n == 0) return VS_OK;
    if (!xs_dev) return set_err(VS_ERR_INVALID, "null vectors");
    if (x->ntotal + n > (int64_t)INT32_MAX)
        return set_err(VS_ERR_INVALID, "ids are int32: ntotal + n must stay below 2^31");
    DeviceGuard g(x->device);
    return add_device_rows(x, xs_dev, src_dtype, n);
}

int vs_index_reconstruct(vs_index *x, int64_t i0, int64_t n, float *out) {
    if (int rc = check_index(x)) return rc;
    if (i0 < 0 || n < 0 || i0 + n > x->ntotal)
        return set_err(VS_ERR_INVALID, "rows [%lld, %lld) out of range [0, %lld)", (long long)i0,
                       (long long)(i0 + n), (long long)x->ntotal);
    if (n == 0) return VS_OK;
    if (!out) return set_err(VS_ERR_INVALID, "null output");
    DeviceGuard g(x->device);
    const int64_t rb = row_bytes(x);
    // rows come through a pinned staging buffer of at most 64 MiB
    const int64_t per = std::max<int64_t>(1, std::min<int64_t>(n, (int64_t)(64 << 20) / rb));
    VS_HIP(x->rstage.ensure((size_t)per * rb), "pinned staging");
    for (int64_t r0 = 0; r0 < n; r0 += per) {
        const int64_t m = std::min(per, n - r0);
        VS_HIP(hipMemcpyAsync(x->rstage.p, (const char *)x->xb + (size_t)(i0 + r0) * rb,
                              (size_t)m * rb, hipMemcpyDeviceToHost, x->st),
               "reading rows");
        VS_HIP(hipStreamSynchronize(x->st), "reading rows");
        const char *src = x->rstage.as<char>();
        float *dst = out + r0 * x->d;
        if (x->storage == 1) {
            for (int64_t r = 0; r < m; ++r) {
                const uint16_t *h = (const uint16_t *)(src + r * rb);
                float *o = dst + r * x->d;
                for (int64_t j = 0; j < x->d; ++j) o[j] = bf16_to_f32(h[j]);
            }
        } else {
            for (int64_t r = 0; r < m; ++r)
                memcpy(dst + r * x->d, src + r * rb, (size_t)x->d * 4);
        }
    }
    return VS_OK;
}

int vs_index_remove_ids(vs_index *x, const int64_t *ids, int64_t n, int64_t *nremoved) {
    if (int rc = check_index(x)) return rc;
    if (n < 0) return set_err(VS_ERR_INVALID, "n must be >= 0");
    if (nremoved) *nremoved = 0;
    if (n == 0 || x->ntotal == 0) return VS_OK;
    if (!ids) return set_err(VS_ERR_INVALID, "null ids");
    DeviceGuard g(x->device);
    std::vector<uint8_t> drop((size_t)x->ntotal, 0);
    for (int64_t t = 0; t < n; ++t)
        if (ids[t] >= 0 && ids[t] < x->ntotal) drop[(size_t)ids[t]] = 1;
    std::vector<int32_t> dst((size_t)x->ntotal);
    int64_t w = 0;
    for (int64_t r = 0; r < x->ntotal; ++r) dst[(size_t)r] = drop[(size_t)r] ? -1 : (int32_t)w++;
    const int64_t removed = x->ntotal - w;
    if (removed == 0) return VS_OK;
    const int64_t rb = row_bytes(x);
    void *nxb = nullptr;
    float *nxn = nullptr;
    const size_t xbytes = (size_t)(x->cap + kRowSlack) * rb;
    const size_t nbytes = (size_t)(x->cap + kRowSlack) * 4;
    VS_HIP(dev_malloc(&nxb, xbytes), "removeIds storage");
    if (dev_malloc((void **)&nxn, nbytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(nxb);
        return set_err(VS_ERR_OOM, "removeIds norms");
    }
    VS_HIP(hipMemsetAsync(nxb, 0, xbytes, x->st), "removeIds");
    VS_HIP(hipMemsetAsync(nxn, 0, nbytes, x->st), "removeIds");
    VS_HIP(x->misc.ensure((size_t)x->ntotal * 4), "removeIds map");
    VS_HIP(hipMemcpyAsync(x->misc.p, dst.data(), (size_t)x->ntotal * 4, hipMemcpyHostToDevice,
                          x->st),
           "removeIds map");
    VS_HIP(vs::launch_compact_rows(x->xb, nxb, x->xn, nxn, x->misc.as<int32_t>(), x->ntotal, rb,
                                   x->st),
           "removeIds compaction");
    VS_HIP(hipStreamSynchronize(x->st), "removeIds");
    (void)hipFree(x->xb);
    (void)hipFree(x->xn);
    x->xb = nxb;
    x->xn = nxn;
    x->ntotal = w;
    ++x->version;
    if (nremoved) *nremoved = removed;
    return VS_OK;
}

int vs_index_search_device(vs_index *x, const void *q_dev, int q_dtype, int64_t nq, int64_t k,
                           float *D_dev, int32_t *I_dev) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(q_dtype)) return rc;
    if (nq > 0 && k > 0 && (!q_dev || !D_dev || !I_dev))
        return set_err(VS_ERR_INVALID, "null query or output buffer");
    DeviceGuard g(x->device);
    Arena A;
    return search_device(x, A, q_dev, q_dtype, nq, k, D_dev, I_dev);
}

int vs_index_search_device_noalloc(vs_index *x, const void *q_dev, int q_dtype, int64_t nq,
                                   int64_t k, float *D_dev, int32_t *I_dev) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(q_dtype)) return rc;
    if (nq < 0 || k < 0) return set_err(VS_ERR_INVALID, "nq and k must be >= 0");
    if (nq > kFixedMaxNq || k > kFixedMaxK || x->d > kFixedMaxD)
        return set_err(VS_ERR_UNSUPPORTED,
                       "allocation-free search: nq <= %lld, k <= %lld, d <= %lld (got nq=%lld, "
                       "k=%lld, d=%lld)",
                       (long long)kFixedMaxNq, (long long)kFixedMaxK, (long long)kFixedMaxD,
                       (long long)nq, (long long)k, (long long)x->d);
    if (nq > 0 && k > 0 && (!q_dev || !D_dev || !I_dev))
        return set_err(VS_ERR_INVALID, "null query or output buffer");
    DeviceGuard g(x->device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    char *base = nullptr;
    if (int rc = fixed_scratch(x->device, &base)) return rc;
    // one call at a time per GPU: the region is shared by every handle on it
    std::lock_guard<std::mutex> lk(g_scratch_call_mu[x->device]);
    Arena A;
    A.base = base;
    A.cap = kFixedScratchBytes;
    struct FixedScope {
        vs_index *x;
        // the region is free again only once this call's GPU work is done,
        // also after an error part-way through
        ~FixedScope() {
            (void)hipStreamSynchronize(x->st);
            x->prof_fixed = false;
        }
    } fs{x};
    x->prof_fixed = true;
    return search_device(x, A, q_dev, q_dtype, nq, k, D_dev, I_dev, false, kFixedListBudget);
}

int vs_index_search(vs_index *x, const void *q, int q_dtype, int64_t nq, int64_t k, float *D,
                    int32_t *I) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(q_dtype)) return rc;
    if (nq < 0 || k < 0) return set_err(VS_ERR_INVALID, "nq and k must be >= 0");
    if (nq == 0) return VS_OK;
    if (k > 0 && (!q || !D || !I)) return set_err(VS_ERR_INVALID, "null query or output buffer");
    DeviceGuard g(x->device);
    const size_t qbytes = (size_t)nq * x->d * (q_dtype == 1 ? 2 : 4);
    VS_HIP(x->stage.ensure(qbytes), "query staging");
    VS_HIP(hipMemcpyAsync(x->stage.p, q, qbytes, hipMemcpyHostToDevice, x->st), "uploading queries");
    Arena A;
    if (k == 0) return search_device(x, A, x->stage.p, q_dtype, nq, k, nullptr, nullptr);
    VS_HIP(x->outD.ensure((size_t)nq * k * 4), "result buffer");
    VS_HIP(x->outI.ensure((size_t)nq * k * 4), "result buffer");
    int rc = search_device(x, A, x->stage.p, q_dtype, nq, k, x->outD.as<float>(),
                           x->outI.as<int32_t>());
    if (rc) return rc;
    VS_HIP(hipMemcpyAsync(D, x->outD.p, (size_t)nq * k * 4, hipMemcpyDeviceToHost, x->st),
           "reading distances");
    VS_HIP(hipMemcpyAsync(I, x->outI.p, (size_t)nq * k * 4, hipMemcpyDeviceToHost, x->st),
           "reading ids");
    VS_HIP(hipStreamSynchronize(x->st), "search");
    return VS_OK;
}

int vs_index_range_search(vs_index *x, const void *q, int q_dtype, int64_t nq, double radius,
                          vs_range_result **out) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(q_dtype)) return rc;
    if (!out) return set_err(VS_ERR_INVALID, "null output");
    *out = nullptr;
    if (nq < 0) return set_err(VS_ERR_INVALID, "nq must be >= 0");
    if (nq > 0 && !q) return set_err(VS_ERR_INVALID, "null queries");
    if (!std::isfinite(radius)) return set_err(VS_ERR_INVALID, "radius must be finite");
    DeviceGuard g(x->device);
    RangeHits hits;
    if (nq > 0 && x->ntotal > 0) {
        const size_t qbytes = (size_t)nq * x->d * (q_dtype == 1 ? 2 : 4);
        VS_HIP(x->stage.ensure(qbytes), "query staging");
        VS_HIP(hipMemcpyAsync(x->stage.p, q, qbytes, hipMemcpyHostToDevice, x->st),
               "uploading queries");
        vs::PreparedQueries pq;
        uint32_t f = 0;
        Arena A;
        int rc = prepare_queries(x, A, x->stage.p, q_dtype, x->d, nq, &pq, &f);
        if (rc) return rc;
        rc = range_core(x, pq, radius, 0, f, &hits);
        if (rc) return rc;
    }
    vs_range_result *r = (vs_range_result *)calloc(1, sizeof(vs_range_result));
    if (!r) return set_err(VS_ERR_OOM, "host allocation");
    const size_t m = hits.q.size();
    r->nq = nq;
    r->lims = (int64_t *)calloc((size_t)nq + 1, sizeof(int64_t));
    r->D = (float *)malloc(std::max<size_t>(m, 1) * sizeof(float));
    r->I = (int32_t *)malloc(std::max<size_t>(m, 1) * sizeof(int32_t));
    if (!r->lims || !r->D || !r->I) {
        vs_range_result_free(r);
        return set_err(VS_ERR_OOM, "host allocation");
    }
    for (size_t t = 0; t < m; ++t) r->lims[hits.q[t] + 1]++;
    for (int64_t qi = 0; qi < nq; ++qi) r->lims[qi + 1] += r->lims[qi];
    if (m) {
        memcpy(r->D, hits.s.data(), m * sizeof(float));
        memcpy(r->I, hits.id.data(), m * sizeof(int32_t));
    }
    *out = r;
    return VS_OK;
}

int vs_index_score_all(vs_index *x, const float *q, float *out) {
    if (int rc = check_index(x)) return rc;
    if (!q || (x->ntotal > 0 && !out)) return set_err(VS_ERR_INVALID, "null query or output");
    if (x->ntotal == 0) return VS_OK;
    DeviceGuard g(x->device);
    Arena A;
    void *pq, *po;
    VS_TAKE(A.tmp((size_t)x->d * 4, &pq, "query"));
    VS_TAKE(A.tmp((size_t)x->ntotal * 4, &po, "scores"));
    for (int64_t j = 0; j < x->d; ++j)
        if (!std::isfinite(q[j])) return set_err(VS_ERR_NONFINITE, "query contains NaN or infinity");
    VS_HIP(hipMemcpyAsync(pq, q, (size_t)x->d * 4, hipMemcpyHostToDevice, x->st), "query upload");
    VS_HIP(vs::launch_exact_all(x->xb, x->storage, x->ld, x->d, x->metric, (const float *)pq,
                                x->ntotal, (float *)po, x->st),
           "exact scores");
    VS_HIP(hipMemcpyAsync(out, po, (size_t)x->ntotal * 4, hipMemcpyDeviceToHost, x->st),
           "scores download");
    VS_HIP(hipStreamSynchronize(x->st), "exact scores");
    return VS_OK;
}

}  // extern "C"

// Subset search beyond the list path's keep (k > 409): per query, the fp64
// score of every row its segments name, as (fp32 key code, id) keys sorted
// on the device (exact_sort_topk_ids); the k first are the answer, sentinel
// padded past the subset's size.  The ids are checked on the host (the
// list path checks them in its kernels).
static int search_subsets_sorted(vs_index *x, Arena &A, const vs::PreparedQueries &pq, int64_t k,
                                 const int32_t *ids, const int64_t *seg_off,
                                 const int64_t *seg_len, int64_t nseg, float *D, int32_t *I) {
    const int64_t nq = pq.nq;
    int64_t mmax = 0;
    for (int64_t qi = 0; qi < nq; ++qi) {
        int64_t m = 0;
        for (int64_t s = 0; s < nseg; ++s) {
            const int64_t o = seg_off[qi * nseg + s], l = seg_len[qi * nseg + s];
            for (int64_t j = o; j < o + l; ++j)
                if (ids[j] < 0 || ids[j] >= x->ntotal)
                    return set_err(VS_ERR_INVALID, "id %lld of query %lld outside [0, %lld)",
                                   (long long)ids[j], (long long)qi, (long long)x->ntotal);
            m += l;
        }
        mmax = std::max(mmax, m);
    }
    if (mmax > (int64_t)UINT32_MAX)
        return set_err(VS_ERR_UNSUPPORTED, "a query's subsets hold %lld rows", (long long)mmax);
    size_t tmp_bytes = 0;
    VS_HIP(vs::exact_sort_topk_ids(x->xb, x->storage, x->ld, x->d, x->metric, pq.qf, nullptr, mmax,
                                   k, nullptr, nullptr, nullptr, nullptr, tmp_bytes, x->st),
           "sort size");
    void *pids, *keys, *tmp, *pD, *pI;
    VS_TAKE(A.tmp((size_t)std::max<int64_t>(mmax, 1) * 4, &pids, "subset ids"));
    VS_TAKE(A.tmp((size_t)std::max<int64_t>(mmax, 1) * 16, &keys, "sort keys"));
    VS_TAKE(A.tmp(tmp_bytes + 256, &tmp, "sort scratch"));
    VS_TAKE(A.tmp((size_t)k * 4, &pD, "results"));
    VS_TAKE(A.tmp((size_t)k * 4, &pI, "results"));
    std::vector<int32_t> flat((size_t)std::max<int64_t>(mmax, 1));
    for (int64_t qi = 0; qi < nq; ++qi) {
        int64_t m = 0;
        for (int64_t s = 0; s < nseg; ++s) {
            const int64_t o = seg_off[qi * nseg + s], l = seg_len[qi * nseg + s];
            std::copy(ids + o, ids + o + l, flat.begin() + m);
            m += l;
        }
        // (flat is refilled only after the stream has finished with it)
        if (m > 0)
            VS_HIP(hipMemcpyAsync(pids, flat.data(), (size_t)m * 4, hipMemcpyHostToDevice, x->st),
                   "ids");
        VS_HIP(vs::exact_sort_topk_ids(x->xb, x->storage, x->ld, x->d, x->metric, pq.qf + qi * x->d,
                                       (const int32_t *)pids, m, k, (float *)pD, (int32_t *)pI,
                                       (uint64_t *)keys, tmp, tmp_bytes, x->st),
               "subset sort");
        VS_HIP(hipMemcpyAsync(D + qi * k, pD, (size_t)k * 4, hipMemcpyDeviceToHost, x->st),
               "results");
        VS_HIP(hipMemcpyAsync(I + qi * k, pI, (size_t)k * 4, hipMemcpyDeviceToHost, x->st),
               "results");
        VS_HIP(hipStreamSynchronize(x->st), "subset search");
    }
    if (!x->prof_fixed) x->prof["exact_sort_queries"].launches += nq;
    return VS_OK;
}

extern "C" {

int vs_index_search_subsets(vs_index *x, const void *q, int q_dtype, int64_t nq, int64_t k,
                            const int32_t *ids, int64_t nids, const int64_t *seg_off,
                            const int64_t *seg_len, int64_t nseg, float *D, int32_t *I) {
    if (int rc = check_index(x)) return rc;
    if (int rc = check_dtype(q_dtype)) return rc;
    if (nq < 0 || k < 0 || nids < 0 || nseg < 0)
        return set_err(VS_ERR_INVALID, "nq, k, nids and nseg must be >= 0");
    if (nq == 0) return VS_OK;
    if (k == 0) return set_err(VS_ERR_INVALID, "k must be >= 1");
    const int64_t kk = std::max<int64_t>(8, next_pow2(k + std::max<int64_t>(4, k / 4)));
    if (k > INT32_MAX) return set_err(VS_ERR_INVALID, "k = %lld is too large", (long long)k);
    if (!q || !D || !I || (nq * nseg > 0 && (!seg_off || !seg_len)) || (nids > 0 && !ids))
        return set_err(VS_ERR_INVALID, "null buffer");
    for (int64_t t = 0; t < nq * nseg; ++t)
        if (seg_off[t] < 0 || seg_len[t] < 0 || seg_off[t] + seg_len[t] > nids)
            return set_err(VS_ERR_INVALID, "segment %lld [%lld, +%lld) outside the %lld ids",
                           (long long)t, (long long)seg_off[t], (long long)seg_len[t],
                           (long long)nids);
    DeviceGuard g(x->device);
    Arena A;
    const size_t qbytes = (size_t)nq * x->d * (q_dtype == 1 ? 2 : 4);
    VS_HIP(x->stage.ensure(qbytes), "query staging");
    VS_HIP(hipMemcpyAsync(x->stage.p, q, qbytes, hipMemcpyHostToDevice, x->st), "uploading queries");
    vs::PreparedQueries pq;
    if (int rc = prepare_queries(x, A, x->stage.p, q_dtype, x->d, nq, &pq, nullptr)) return rc;
    if (kk > 512) return search_subsets_sorted(x, A, pq, k, ids, seg_off, seg_len, nseg, D, I);
    const int64_t ns = std::max<int64_t>(1, nseg);
    void *pids, *poff, *plen, *pv, *pi, *pf, *pD, *pI;
    VS_TAKE(A.tmp((size_t)std::max<int64_t>(nids, 1) * 4, &pids, "ids"));
    VS_TAKE(A.tmp((size_t)nq * ns * 8, &poff, "segments"));
    VS_TAKE(A.tmp((size_t)nq * ns * 8, &plen, "segments"));
    VS_TAKE(A.tmp((size_t)nq * ns * kk * 4, &pv, "lists"));
    VS_TAKE(A.tmp((size_t)nq * ns * kk * 4, &pi, "lists"));
    VS_TAKE(A.tmp(4, &pf, "flags"));
    VS_TAKE(A.tmp((size_t)nq * k * 4, &pD, "results"));
    VS_TAKE(A.tmp((size_t)nq * k * 4, &pI, "results"));
    if (nids > 0)
        VS_HIP(hipMemcpyAsync(pids, ids, (size_t)nids * 4, hipMemcpyHostToDevice, x->st), "ids");
    if (nseg > 0) {
        VS_HIP(hipMemcpyAsync(poff, seg_off, (size_t)nq * nseg * 8, hipMemcpyHostToDevice, x->st),
               "segments");
        VS_HIP(hipMemcpyAsync(plen, seg_len, (size_t)nq * nseg * 8, hipMemcpyHostToDevice, x->st),
               "segments");
    } else {  // one empty segment per query
        VS_HIP(vs::launch_fill32(poff, nq * 2, 0u, x->st), "segments");
        VS_HIP(vs::launch_fill32(plen, nq * 2, 0u, x->st), "segments");
    }
    VS_HIP(vs::launch_fill32(pf, 1, 0u, x->st), "flags");
    VS_HIP(vs::launch_exact_lists(x->xb, x->storage, x->ld, x->d, x->metric, pq.qf, nq, x->ntotal,
                                  (int)kk, ns, 0, (float *)pv, (int32_t *)pi, x->st,
                                  (const int32_t *)pids, (const int64_t *)poff,
                                  (const int64_t *)plen, (uint32_t *)pf),
           "subset lists");
    vs::ScanPlan plan;
    plan.kind = 0;
    plan.bn = 1;
    plan.lw = 1;
    plan.kk = (int)kk;
    plan.kk_final = (int)kk;
    plan.cap = (int)kk;
    plan.nqblk = nq;
    plan.nsplit = ns;
    VS_HIP(vs::launch_merge_refine(x->xb, x->storage, x->ld, x->d, x->metric, pq, plan,
                                   (float *)pv, (int32_t *)pi, nullptr, nullptr, nullptr, nullptr,
                                   k, (float *)pD, (int32_t *)pI, x->ntotal, (uint32_t *)pf, 0,
                                   nullptr, nullptr, x->st),
           "subset merge");
    uint32_t f = 0;
    VS_HIP(hipMemcpyAsync(&f, pf, 4, hipMemcpyDeviceToHost, x->st), "flags");
    VS_HIP(hipMemcpyAsync(D, pD, (size_t)nq * k * 4, hipMemcpyDeviceToHost, x->st), "results");
    VS_HIP(hipMemcpyAsync(I, pI, (size_t)nq * k * 4, hipMemcpyDeviceToHost, x->st), "results");
    VS_HIP(hipStreamSynchronize(x->st), "subset search");
    if (f & vs::kFlagBadId) return set_err(VS_ERR_INVALID, "an id in the lists is outside [0, ntotal)");
    return VS_OK;
}

void vs_range_result_free(vs_range_result *r) {
    if (!r) return;
    free(r->lims);
    free(r->D);
    free(r->I);
    free(r);
}

int vs_index_self_join(vs_index *x, double threshold, vs_pairs **out) {
    if (int rc = check_index(x)) return rc;
    if (!out) return set_err(VS_ERR_INVALID, "null output");
    *out = nullptr;
    if (!std::isfinite(threshold)) return set_err(VS_ERR_INVALID, "threshold must be finite");
    DeviceGuard g(x->device);
    RangeHits hits;
    if (x->ntotal > 1) {
        vs::PreparedQueries pq;
        uint32_t f = 0;
        Arena A;
        int rc = prepare_queries(x, A, x->xb, x->storage, x->ld, x->ntotal, &pq, &f);
        if (rc) return rc;
        rc = range_core(x, pq, threshold, 1, f, &hits);
        if (rc) return rc;
    }
    vs_pairs *p = (vs_pairs *)calloc(1, sizeof(vs_pairs));
    if (!p) return set_err(VS_ERR_OOM, "host allocation");
    const size_t m = hits.q.size();
    p->npairs = (int64_t)m;
    p->i = (int32_t *)malloc(std::max<size_t>(m, 1) * 4);
    p->j = (int32_t *)malloc(std::max<size_t>(m, 1) * 4);
    p->s = (float *)malloc(std::max<size_t>(m, 1) * 4);
    if (!p->i || !p->j || !p->s) {
        vs_pairs_free(p);
        return set_err(VS_ERR_OOM, "host allocation");
    }
    if (m) {
        memcpy(p->i, hits.q.data(), m * 4);
        memcpy(p->j, hits.id.data(), m * 4);
        memcpy(p->s, hits.s.data(), m * 4);
    }
    *out = p;
    return VS_OK;
}

void vs_pairs_free(vs_pairs *p) {
    if (!p) return;
    free(p->i);
    free(p->j);
    free(p->s);
    free(p);
}

int vs_kmeans_step(vs_index *x, const float *centroids_in, int64_t K, int64_t min_points,
                   const double *jitter_u, int64_t njitter, int32_t *assign, float *centroids_out,
                   int32_t *counts, double *obj) {
    if (int rc = check_index(x)) return rc;
    if (K <= 0) return set_err(VS_ERR_INVALID, "K must be > 0");
    if (!centroids_in || !assign || !centroids_out || !counts)
        return set_err(VS_ERR_INVALID, "null buffer");
    if (njitter < 0 || (njitter > 0 && !jitter_u))
        return set_err(VS_ERR_INVALID, "bad jitter buffer");
    if (x->storage != 0)
        return set_err(VS_ERR_UNSUPPORTED, "k-means points must use fp32 storage");
    if (x->ntotal < K)
        return set_err(VS_ERR_INVALID, "k-means: need at least k=%lld vectors, got %lld",
                       (long long)K, (long long)x->ntotal);
    if (K > (int64_t)INT32_MAX) return set_err(VS_ERR_INVALID, "K too large");
    DeviceGuard g(x->device);
    Arena A;
    const int64_t n = x->ntotal, d = x->d, ld = x->ld;
    // the input centroids are read again at the end (empty clusters); a copy
    // only when the output may overwrite them first
    const size_t cbytes = (size_t)K * d * 4;
    const bool alias = (const char *)centroids_out < (const char *)centroids_in + cbytes &&
                       (const char *)centroids_in < (const char *)centroids_out + cbytes;
    std::vector<float> cen_copy;
    if (alias) cen_copy.assign(centroids_in, centroids_in + K * d);
    const float *cen_in = alias ? cen_copy.data() : centroids_in;

    // the previous step's results, if they belong to these points and K:
    // how far each centroid moved since (before its rows are replaced)
    const bool prev = x->km_prev_version == x->version && x->km_prev_n == n && x->km_prev_K == K;
    x->km_prev_version = ~0ull;  // set again once this step's results are whole
    VS_HIP(x->stage.ensure((size_t)K * d * 4), "centroid staging");
    VS_HIP(hipMemcpyAsync(x->stage.p, cen_in, (size_t)K * d * 4, hipMemcpyHostToDevice,
                          x->st),
           "uploading centroids");
    if (prev) {
        VS_HIP(x->km_shift.ensure((size_t)K * 8), "centroid shifts");
        VS_HIP(vs::launch_kmeans_shift(x->km_cen.as<float>(), ld, (const float *)x->stage.p, d, K,
                                       x->km_shift.as<double>(), x->st),
               "centroid shifts");
    }
    // centroid storage: fp32 rows of ld, slack rows zero, plus norms
    VS_HIP(x->km_cen.ensure((size_t)(K + kRowSlack) * ld * 4), "centroid storage");
    VS_HIP(x->km_cxn.ensure((size_t)(K + kRowSlack) * 4), "centroid norms");
    VS_HIP(hipMemsetAsync(x->km_cen.p, 0, (size_t)(K + kRowSlack) * ld * 4, x->st), "clear");
    VS_HIP(hipMemsetAsync(x->km_cxn.p, 0, (size_t)(K + kRowSlack) * 4, x->st), "clear");
    // misc: [0] the largest centroid norm, [1] the centroids' flags, [2] the
    // accumulator bound -- all on the device: no host round trip separates
    // the centroids from the assign scan (the flags are read with the
    // pick's results, before any exhaustive pass)
    VS_HIP(x->misc.ensure(16), "misc");
    float *kmisc = x->misc.as<float>();
    uint32_t *cflags_dev = (uint32_t *)(kmisc + 1);
    VS_HIP(vs::launch_fill32(cflags_dev, 1, 0u, x->st), "flags");
    VS_HIP(vs::launch_store_rows(x->stage.p, 0, d, K, d, x->km_cen.p, 0, ld,
                                 x->km_cxn.as<float>(), cflags_dev, x->st),
           "storing centroids");
    VS_HIP(vs::launch_max_reduce(x->km_cxn.as<float>(), K, kmisc, x->st), "max");
    VS_HIP(x->flags.ensure(4), "flags");

    // points as prepared queries against the centroid "database" (kept
    // across iterations while the stored rows are unchanged)
    if (x->km_prep_version != x->version) {
        x->km_prep_version = ~0ull;
        int rc0 = prepare_queries(x, A, x->xb, 0, ld, n, &x->km_pq, &x->km_pflags, x->km_qp,
                                  x->km_qf, x->km_qnorm);
        if (rc0) return rc0;
        x->km_prep_version = x->version;
    }
    const vs::PreparedQueries pq = x->km_pq;
    int rc = VS_OK;
    // the distance kernels index the centroid rows with the points' ld
    vs_index cview;
    cview.ld = ld;
    cview.d = d;
    cview.lds_max = x->lds_max;
    cview.num_cu = x->num_cu;
    cview.opt = x->opt;
    // one-pass selection (bf16 hi planes of points and centroids) where the
    // GEMM-tiled scan runs it; the shortlist proof below widens its bound
    vs::ScanPlan plan;
    bool coarse = x->opt.coarse != 0;
    if (coarse) coarse = plan_scan(&cview, n, K, 1, 16, vs::kSelectCoarse, &plan) == VS_OK &&
                         (plan.kind == 2 || plan.kind == 3);
    if (!coarse) {
        plan = vs::ScanPlan();
        rc = plan_scan(&cview, n, K, pq.planes, 16, 0, &plan);
        if (rc) return rc;
    }
    float pmax = 0.f;
    VS_TAKE(xnorm_max(x, A, &pmax));
    // Error of the accumulator |c|^2 - 2 x.c (point x, centroid c):
    //  - operands: each product of the MFMA operands lies within r |2 x_j c_j|
    //    of -2 x_j c_j, r = 2^-8 for the one-pass selection (both operands
    //    rounded to bf16, 2^-9 each) and 2^-15 for the split-bf16 passes (hi
    //    + lo within 2^-18 of each value, the dropped lo * q1 term);
    //  - fp32 accumulation (accum_gamma) of one pass (one-pass selection) or
    //    of three (split-bf16 points and centroids);
    // so |error| <= 2 r |x| |c| + gamma (|c|^2 + 2 |x| |c|) (Cauchy-Schwarz),
    // taken with a 25% margin.
    const double r = coarse ? 1.0 / 256.0 : 1.0 / 32768.0;
    const double gam = accum_gamma(d, coarse ? 1 : 3);
    float *bound_dev = kmisc + 2;
    VS_HIP(vs::launch_kmeans_bound(kmisc, (double)pmax, r, gam, bound_dev, x->st), "bound");
    plan.dev_bound = bound_dev;
    const float bound = 0.f;  // (the kernels read bound_dev)
    // On the row-shared scan each lane appends every value below its running
    // minimum + 2.5 bound to its list (the pick re-scores those within 2 bound
    // of the smallest and proves the rest worse with the other half bound).
    if (coarse && plan.kind == 3) {
        plan.share_kmin = 1;
        plan.kmin_margin = 0.f;  // 2.5 * bound_dev, read by the kernels
        // option km16_nqb 4: 64 points per wave on the bf16 copy of the
        // centroids (32-row tiles keep it at two waves per SIMD); decided
        // here, before the lists are sized
        if (x->opt.km16_nqb == 4 && x->opt.km16 && plan.tile_st == vs::kSelectCoarse &&
            plan.nks == 8) {
            const size_t lds = vs::share_lds_bytes(plan.nks, 4, 2, plan.cap, 1);
            if (lds <= x->lds_max) {
                plan.bn = 256;
                plan.tm = 2;
                plan.lds_bytes = lds;
                plan.nqblk = (n + plan.bn - 1) / plan.bn;
            }
        }
        // the running minima start at the previous assignment's bound
        if (prev && x->opt.kmin_init) {
            VS_HIP(x->km_init.ensure((size_t)pq.nq_pad * 4), "running minima");
            VS_HIP(vs::launch_kmeans_init(x->km_assign.as<int32_t>(), x->km_best.as<double>(),
                                          x->km_shift.as<double>(), pq.qnorm, n, pq.nq_pad, K,
                                          bound, bound_dev, x->km_init.as<float>(), x->st),
                   "running minima");
            plan.kmin_init = x->km_init.as<float>();
            x->prof["kmin_init"].launches++;
        }
        // the points grouped by the previous step's clusters (the order the
        // update sorted them into): a wave's points then share their few
        // candidate centroids, so most row blocks append nothing
        if (x->opt.assign_order && x->km_order_version == x->version && x->km_order_n == n) {
            plan.qorder = x->km_order.as<int32_t>();
            x->prof["assign_order"].launches++;
        }
    }
    if ((rc = scan_fits(plan, pq))) return rc;
    const size_t nlists = (size_t)plan.nqblk * plan.nsplit * plan.lw * plan.bn;
    const size_t nlist = nlists * plan.cap;
    VS_HIP(x->cand_v.ensure(nlist * 4), "candidate lists");
    VS_HIP(x->cand_i.ensure(nlist * 4), "candidate lists");
    VS_HIP(x->lcnt.ensure((nlists + 1) * 4), "list counts");
    VS_HIP(hipMemsetAsync(x->lcnt.as<int32_t>() + nlists, 0, 4, x->st), "list counts");
    VS_HIP(x->gthr.ensure((size_t)pq.nq_pad * 4), "shared thresholds");
    VS_HIP(hipMemsetD32Async((hipDeviceptr_t)x->gthr.p, (int)vs::kGthrInit, (size_t)pq.nq_pad, x->st),
           "shared thresholds");
    // the one-pass selection multiplies the bf16 rounding of the centroids:
    // the row-shared scan reads a bf16 copy of them (half the bytes of the
    // fp32 rows it would round itself) with the fp32 rows' norms
    const void *scan_rows = x->km_cen.p;
    int scan_storage = 0;
    if (plan.kind == 3 && plan.share_kmin && plan.tile_st == vs::kSelectCoarse && plan.nks == 8 &&
        x->opt.km16) {
        VS_HIP(x->km_cen16.ensure((size_t)(K + kRowSlack) * ld * 2), "centroid copy");
        VS_HIP(x->km_c16n.ensure((size_t)(K + kRowSlack) * 4), "centroid copy");
        VS_HIP(hipMemsetAsync(x->km_cen16.p, 0, (size_t)(K + kRowSlack) * ld * 2, x->st), "clear");
        VS_HIP(vs::launch_store_rows(x->km_cen.p, 0, ld, K, ld, x->km_cen16.p, 1, ld,
                                     x->km_c16n.as<float>(), x->flags.as<uint32_t>(), x->st),
               "centroid copy");
        plan.tile_st = 1;
        // bf16 rows stage twice the rows per tile in the same registers
        const int rt = x->opt.km16_rt;
        if (rt == 4 && plan.bn == 128) {
            const size_t lds = vs::share_lds_bytes(plan.nks, plan.bn / 64, 4, plan.cap, 1);
            if (lds <= x->lds_max) {
                plan.tm = 4;
                plan.lds_bytes = lds;
                plan.rows_per_split = round_up(plan.rows_per_split, 64);
                plan.nsplit = std::max<int64_t>(1, (K + plan.rows_per_split - 1) / plan.rows_per_split);
            }
        }
        scan_rows = x->km_cen16.p;
        scan_storage = 1;
    }
    note_scan_kind(x, plan);
    {
        ProfScope ps(x, "assign");
        VS_HIP(vs::launch_scan_topk(scan_rows, scan_storage, ld, x->km_cxn.as<float>(), K, 0, pq, plan,
                                    x->cand_v.as<float>(), x->cand_i.as<int32_t>(),
                                    x->gthr.as<uint32_t>(), nullptr, x->lcnt.as<int32_t>(), x->st),
               "assign scan");
    }

    VS_HIP(x->km_assign.ensure((size_t)n * 4), "assignments");
    VS_HIP(x->km_best.ensure((size_t)n * 8), "distances");
    VS_HIP(x->km_fb.ensure((size_t)(n + 1) * 4), "fallback list");
    VS_HIP(hipMemsetAsync(x->km_fb.p, 0, 4, x->st), "fallback count");
    int32_t *fb_count = x->km_fb.as<int32_t>();
    int32_t *fb_list = fb_count + 1;
    VS_HIP(hipMemsetAsync(x->flags.p, 0, sizeof(uint32_t), x->st), "clearing flags");
    // distances and assignments go to pinned memory on a second stream, so
    // that the copies overlap the GPU's later work
    constexpr int kSumChunks = 4;
    VS_HIP(x->km_hbest.ensure((size_t)n * 8), "pinned distances");
    VS_HIP(x->km_hassign.ensure((size_t)n * 4), "pinned assignments");
    VS_HIP(x->km_hcen.ensure((size_t)K * d * 4), "pinned centroids");
    VS_HIP(x->km_hfb.ensure((size_t)kSumChunks * 4), "pinned fallback counts");
    if (!x->st_copy)
        VS_HIP(hipStreamCreateWithFlags(&x->st_copy, hipStreamNonBlocking), "copy stream");
    // The objective is a sequential fp64 sum over the points in index order
    // (kmeans.dart:104): a chain of n dependent adds on the host.  Over the
    // row-shared scan's lists the pick runs in kSumChunks launches over
    // consecutive point ranges (each range's points in the previous step's
    // grouped order), and each range's distances and assignments come over
    // with the fallback count so far as soon as its pick ends: the sum of a
    // range, and the copy of its assignments into the caller's buffer, run
    // while the GPU picks the next ones.  From the first range with a
    // fallback point on, both wait for the exhaustive pass.
    struct EvGuard {
        hipEvent_t e = nullptr;
        ~EvGuard() {
            if (e) (void)hipEventDestroy(e);
        }
    } ev_pick[kSumChunks], ev_best[kSumChunks], ev_fix;
    for (auto &e : ev_pick) VS_HIP(hipEventCreateWithFlags(&e.e, hipEventDisableTiming), "event");
    for (auto &e : ev_best) VS_HIP(hipEventCreateWithFlags(&e.e, hipEventDisableTiming), "event");
    VS_HIP(hipEventCreateWithFlags(&ev_fix.e, hipEventDisableTiming), "event");
    // the copy stream is drained before this call returns (below, and on
    // every error path), so the next call cannot overwrite what it reads
    struct CopyDrain {
        hipStream_t s;
        ~CopyDrain() { (void)hipStreamSynchronize(s); }
    } drain{x->st_copy};
    const bool chunked = plan.kind == 3 && plan.share_kmin;
    const int32_t *order = x->km_order_version == x->version && x->km_order_n == n &&
                                   x->opt.pick_order
                               ? x->km_order.as<int32_t>()
                               : nullptr;
    if (chunked && order) {
        // each range's points in walk order at that same range: a stable
        // partition of the order by range
        VS_HIP(x->km_pkeys.ensure((size_t)n * 4), "range keys");
        VS_HIP(x->km_part.ensure((size_t)n * 4), "range order");
        VS_HIP(x->km_keys.ensure((size_t)n * 4), "sort keys");
        VS_HIP(vs::launch_chunk_keys(order, n, kSumChunks, x->km_pkeys.as<int32_t>(), x->st),
               "range keys");
        size_t pbytes = 0;
        VS_HIP(vs::sort_pairs_by_key(nullptr, pbytes, x->km_pkeys.as<int32_t>(),
                                     x->km_keys.as<int32_t>(), order, x->km_part.as<int32_t>(), n,
                                     2, x->st),
               "sort size");
        VS_HIP(x->km_tmp.ensure(pbytes + 16), "sort scratch");
        VS_HIP(vs::sort_pairs_by_key(x->km_tmp.p, pbytes, x->km_pkeys.as<int32_t>(),
                                     x->km_keys.as<int32_t>(), order, x->km_part.as<int32_t>(), n,
                                     2, x->st),
               "range order");
        order = x->km_part.as<int32_t>();
    }
    {
        ProfScope ps(x, "pick");
        const int npick = chunked ? kSumChunks : 1;
        for (int c = 0; c < npick; ++c) {
            const int64_t s0 = n * c / npick, s1 = n * (c + 1) / npick;
            VS_HIP(vs::launch_kmeans_pick((const float *)x->xb, ld, d, n, x->km_cen.as<float>(), K,
                                          x->cand_v.as<float>(), x->cand_i.as<int32_t>(),
                                          x->gthr.as<uint32_t>(), plan, bound, pq.qf,
                                          x->km_assign.as<int32_t>(), x->km_best.as<double>(),
                                          fb_count, fb_list, x->flags.as<uint32_t>(),
                                          x->lcnt.as<int32_t>(), order ? order + s0 : nullptr,
                                          x->st, s0, s1 - s0),
                   "assign pick");
            VS_HIP(hipEventRecord(ev_pick[c].e, x->st), "event");
        }
    }
    int32_t *hfb = x->km_hfb.as<int32_t>();
    for (int c = 0; c < kSumChunks; ++c) {
        const int64_t i0 = n * c / kSumChunks, i1 = n * (c + 1) / kSumChunks;
        VS_HIP(hipStreamWaitEvent(x->st_copy, ev_pick[chunked ? c : 0].e, 0), "event");
        if (i1 > i0) {
            VS_HIP(hipMemcpyAsync(x->km_hbest.as<double>() + i0, x->km_best.as<double>() + i0,
                                  (size_t)(i1 - i0) * 8, hipMemcpyDeviceToHost, x->st_copy),
                   "reading distances");
            VS_HIP(hipMemcpyAsync(x->km_hassign.as<int32_t>() + i0,
                                  x->km_assign.as<int32_t>() + i0, (size_t)(i1 - i0) * 4,
                                  hipMemcpyDeviceToHost, x->st_copy),
                   "reading assignments");
        }
        VS_HIP(hipMemcpyAsync(hfb + c, fb_count, 4, hipMemcpyDeviceToHost, x->st_copy),
               "reading fallback counts");
        VS_HIP(hipEventRecord(ev_best[c].e, x->st_copy), "event");
    }
    // the sum and the assignments, on a helper thread, up to the first range
    // with a fallback point (`dirty`; the rest follow here after the
    // exhaustive pass)
    double o = 0.0;
    int dirty = kSumChunks;
    hipError_t sum_err = hipSuccess;
    struct Join {
        std::thread t;
        ~Join() {
            if (t.joinable()) t.join();
        }
    } sum_thread{std::thread([&o, &dirty, &sum_err, &ev_best, hfb, assign,
                              best = x->km_hbest.as<double>(),
                              hassign = x->km_hassign.as<int32_t>(), n] {
        double acc = 0.0;
        for (int c = 0; c < kSumChunks; ++c) {
            const hipError_t e = hipEventSynchronize(ev_best[c].e);
            if (e != hipSuccess) {
                sum_err = e;
                return;
            }
            if (hfb[c] > 0) {
                dirty = c;
                break;
            }
            const int64_t i0 = n * c / kSumChunks, i1 = n * (c + 1) / kSumChunks;
            for (int64_t i = i0; i < i1; ++i) acc += best[i];
            memcpy(assign + i0, hassign + i0, (size_t)(i1 - i0) * 4);
        }
        o = acc;
    })};

    int32_t nfb = 0;
    uint32_t pflags = 0, cf = 0;
    VS_HIP(hipMemcpyAsync(&nfb, fb_count, 4, hipMemcpyDeviceToHost, x->st), "fallbacks");
    VS_HIP(hipMemcpyAsync(&pflags, x->flags.p, 4, hipMemcpyDeviceToHost, x->st), "pick flags");
    VS_HIP(hipMemcpyAsync(&cf, cflags_dev, 4, hipMemcpyDeviceToHost, x->st), "centroid flags");
    VS_HIP(hipStreamSynchronize(x->st), "assign");
    if (cf & vs::kFlagNonFinite) return set_err(VS_ERR_NONFINITE, "centroids contain NaN or infinity");
    if (pflags & vs::kFlagBadId)
        return set_err(VS_ERR_HIP, "internal error: a k-means candidate outside the centroids");
    x->prof["kmeans_fallback_points"].launches += nfb;
    int64_t refetch = n;  // distances from here on are read again after the exhaustive pass
    if (nfb > 0) {
        {
            ProfScope ps(x, "exhaustive");
            VS_HIP(vs::launch_kmeans_exhaustive((const float *)x->xb, ld, d,
                                                x->km_cen.as<float>(), K, fb_list, nfb,
                                                x->km_assign.as<int32_t>(),
                                                x->km_best.as<double>(), x->st),
                   "exhaustive assign");
        }
        // the ranges' fallback counts are all in (the sum thread stops at
        // the first nonzero one, and never reads past it)
        VS_HIP(hipEventSynchronize(ev_best[kSumChunks - 1].e), "reading fallback counts");
        int first = 0;
        while (first < kSumChunks && hfb[first] == 0) ++first;
        refetch = n * first / kSumChunks;
    }
    if (refetch < n) {
        VS_HIP(hipEventRecord(ev_fix.e, x->st), "event");
        VS_HIP(hipStreamWaitEvent(x->st_copy, ev_fix.e, 0), "event");
        VS_HIP(hipMemcpyAsync(x->km_hbest.as<double>() + refetch,
                              x->km_best.as<double>() + refetch, (size_t)(n - refetch) * 8,
                              hipMemcpyDeviceToHost, x->st_copy),
               "reading distances");
        VS_HIP(hipMemcpyAsync(x->km_hassign.as<int32_t>() + refetch,
                              x->km_assign.as<int32_t>() + refetch, (size_t)(n - refetch) * 4,
                              hipMemcpyDeviceToHost, x->st_copy),
               "reading assignments");
    }

    // update: counts, stable grouping by cluster, ordered fp32 sums
    VS_HIP(x->km_counts.ensure((size_t)K * 4), "counts");
    VS_HIP(hipMemsetAsync(x->km_counts.p, 0, (size_t)K * 4, x->st), "counts");
    VS_HIP(vs::launch_kmeans_count(x->km_assign.as<int32_t>(), n, K, x->km_counts.as<int32_t>(),
                                   x->st),
           "counts");
    {
        // the point indices 0 .. n - 1 (the sort's values), kept across steps
        void *before = x->km_iota.p;
        VS_HIP(x->km_iota.ensure((size_t)n * 4), "iota");
        if (x->km_iota.p != before || x->km_iota_n != n) {
            std::vector<int32_t> iota((size_t)n);
            std::iota(iota.begin(), iota.end(), 0);
            VS_HIP(hipMemcpyAsync(x->km_iota.p, iota.data(), (size_t)n * 4, hipMemcpyHostToDevice,
                                  x->st),
                   "iota");
            VS_HIP(hipStreamSynchronize(x->st), "iota");
            x->km_iota_n = n;
        }
    }
    VS_HIP(x->km_keys.ensure((size_t)n * 4), "sort keys");
    VS_HIP(x->km_order.ensure((size_t)n * 4), "sort values");
    int key_bits = 1;
    while ((int64_t(1) << key_bits) < K) ++key_bits;
    size_t tmp_bytes = 0;
    VS_HIP(vs::sort_pairs_by_key(nullptr, tmp_bytes, x->km_assign.as<int32_t>(),
                                 x->km_keys.as<int32_t>(), x->km_iota.as<int32_t>(),
                                 x->km_order.as<int32_t>(), n, key_bits, x->st),
           "sort size");
    VS_HIP(x->km_tmp.ensure(tmp_bytes + 16), "sort scratch");
    VS_HIP(vs::sort_pairs_by_key(x->km_tmp.p, tmp_bytes, x->km_assign.as<int32_t>(),
                                 x->km_keys.as<int32_t>(), x->km_iota.as<int32_t>(),
                                 x->km_order.as<int32_t>(), n, key_bits, x->st),
           "grouping points");
    x->km_order_version = x->version;
    x->km_order_n = n;
    VS_HIP(x->km_offsets.ensure((size_t)K * 4), "offsets");
    VS_HIP(vs::launch_exclusive_scan_i32(x->km_counts.as<int32_t>(), K,
                                         x->km_offsets.as<int32_t>(), x->st),
           "offsets");
    // the update starts from the input centroids (the stored rows, d of ld)
    VS_HIP(x->km_out.ensure((size_t)K * d * 4), "new centroids");
    VS_HIP(hipMemcpy2DAsync(x->km_out.p, (size_t)d * 4, x->km_cen.p, (size_t)ld * 4, (size_t)d * 4,
                            (size_t)K, hipMemcpyDeviceToDevice, x->st),
           "new centroids");
    {
        ProfScope ps(x, "update");
        VS_HIP(vs::launch_kmeans_update((const float *)x->xb, ld, d, n, x->km_order.as<int32_t>(),
                                        x->km_offsets.as<int32_t>(), K,
                                        x->km_counts.as<int32_t>(), min_points,
                                        x->km_out.as<float>(), x->st),
               "update");
    }
    VS_HIP(hipMemcpyAsync(x->km_hcen.p, x->km_out.p, (size_t)K * d * 4, hipMemcpyDeviceToHost,
                          x->st),
           "reading centroids");
    VS_HIP(hipMemcpyAsync(counts, x->km_counts.p, (size_t)K * 4, hipMemcpyDeviceToHost, x->st),
           "reading counts");
    VS_HIP(hipStreamSynchronize(x->st), "update");

    // empty clusters, in centroid order, in place (kmeans.dart:127-139): the
    // largest cluster's centroid holds its new value when it precedes c, and
    // still its old one otherwise (c itself included)
    // (the loop changes no count, so the largest cluster -- the first of the
    // largest count -- is the same for every empty one)
    int64_t big = 0, nempty = 0;
    for (int64_t cc = 1; cc < K; ++cc)
        if (counts[cc] > counts[big]) big = cc;
    for (int64_t c = 0; c < K; ++c) nempty += counts[c] < min_points ? 1 : 0;
    if (nempty * d > njitter)
        return set_err(VS_ERR_INVALID, "empty cluster needs more jitter values than the %lld given",
                       (long long)njitter);
    // the new centroids straight into the caller's buffer (an input it
    // aliases was copied above)
    float *cen_new = centroids_out;
    memcpy(cen_new, x->km_hcen.p, (size_t)K * d * 4);
    int64_t used = 0;
    for (int64_t c = 0; c < K; ++c) {
        if (counts[c] >= min_points) continue;
        const float *src = big < c ? &cen_new[(size_t)(big * d)] : &cen_in[(size_t)(big * d)];
        for (int64_t j = 0; j < d; ++j) {
            const double jit = (jitter_u[used++] - 0.5) * 1e-4;
            cen_new[(size_t)(c * d + j)] = (float)((double)src[j] + jit);
        }
    }
    sum_thread.t.join();
    VS_HIP(sum_err, "reading distances");
    if (dirty < kSumChunks) {  // the ranges after the exhaustive pass
        VS_HIP(hipStreamSynchronize(x->st_copy), "reading distances");
        const double *best = x->km_hbest.as<double>();
        const int64_t i0 = n * dirty / kSumChunks;
        double acc = o;
        for (int64_t i = i0; i < n; ++i) acc += best[i];
        o = acc;
        memcpy(assign + i0, x->km_hassign.as<int32_t>() + i0, (size_t)(n - i0) * 4);
    }
    if (obj) *obj = o;
    x->km_prev_version = x->version;
    x->km_prev_n = n;
    x->km_prev_K = K;
    return VS_OK;
}

// ---- flat index files (FAISDART kind 0x01, FAISS IxF2 / IxFI / IxFl) ----

}  // extern "C"

namespace {

// Sequential little-endian reader over a file or a caller's buffer.
struct BlobReader {
    FILE *f = nullptr;
    const unsigned char *buf = nullptr;
    int64_t len = 0, pos = 0;
    ~BlobReader() {
        if (f) fclose(f);
    }
    // reads n bytes; false at end of data
    bool read(void *dst, int64_t n) {
        if (n <= 0) return true;
        if (f) {
            if (fread(dst, 1, (size_t)n, f) != (size_t)n) return false;
            pos += n;
            return true;
        }
        if (pos + n > len) return false;
        memcpy(dst, buf + pos, (size_t)n);
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T *v) {
        return read(v, sizeof(T));
    }
};

// Parses the header (d, metric code of this library, ntotal, is_trained)
// and leaves the reader at the first fp32 of the row-major payload.
//   FAISDART (index_io.dart:8-26, IndexFlat.readFrom index_flat.dart:176-188):
//     'FAISDART', u32 version 1, u32 kind 0x01, u32 d, u32 metric (0 L2 /
//     1 IP), u32 ntotal, u8 isTrained, ntotal * d fp32;
//   FAISS (readFaissIndex, faiss_io.dart:1690-1716; header :419-440):
//     fourcc 'IxF2' / 'IxFI' / 'IxFl', i32 d, i64 ntotal, i64, i64, u8
//     is_trained, i32 metric (FAISS codes 0 IP / 1 L2), u64 byte count
//     (= ntotal * d * 4), the rows.
int parse_flat_header(BlobReader &r, int64_t *d, int *metric, int64_t *ntotal, int *trained) {
    unsigned char magic[8];
    if (!r.read(magic, 4)) return set_err(VS_ERR_INVALID, "truncated index blob (no magic)");
    if (memcmp(magic, "IxF2", 4) == 0 || memcmp(magic, "IxFI", 4) == 0 ||
        memcmp(magic, "IxFl", 4) == 0) {
        int32_t dd = 0, fm = 0;
        int64_t nt = 0, dummy = 0;
        uint8_t tr = 0;
        uint64_t nbytes = 0;
        if (!r.get(&dd) || !r.get(&nt) || !r.get(&dummy) || !r.get(&dummy) || !r.get(&tr) ||
            !r.get(&fm) || !r.get(&nbytes))
            return set_err(VS_ERR_INVALID, "truncated FAISS IndexFlat header");
        if (fm != 0 && fm != 1)
            return set_err(VS_ERR_INVALID, "Unsupported FAISS metric code %d", (int)fm);
        if (dd <= 0 || nt < 0) return set_err(VS_ERR_INVALID, "bad FAISS header: d=%d ntotal=%lld",
                                              (int)dd, (long long)nt);
        if ((int64_t)nbytes != nt * dd * 4)
            return set_err(VS_ERR_INVALID, "IndexFlat payload size %llu != ntotal*d*4 = %lld",
                           (unsigned long long)nbytes, (long long)(nt * dd * 4));
        *d = dd;
        *metric = fm == 1 ? VS_METRIC_L2 : VS_METRIC_IP;
        *ntotal = nt;
        *trained = tr != 0;
        return VS_OK;
    }
    if (!r.read(magic + 4, 4) || memcmp(magic, "FAISDART", 8) != 0)
        return set_err(VS_ERR_INVALID, "not a FAISDART or FAISS IndexFlat blob (bad magic)");
    uint32_t version = 0, kind = 0, dd = 0, m = 0, nt = 0;
    uint8_t tr = 0;
    if (!r.get(&version) || !r.get(&kind))
        return set_err(VS_ERR_INVALID, "truncated FAISDART header");
    if (version != 1) return set_err(VS_ERR_INVALID, "unsupported FAISDART version %u", version);
    if (kind != 0x01) return set_err(VS_ERR_UNSUPPORTED, "FAISDART kind %#x is not IndexFlat", kind);
    if (!r.get(&dd) || !r.get(&m) || !r.get(&nt) || !r.get(&tr))
        return set_err(VS_ERR_INVALID, "truncated FAISDART header");
    if (m > 1) return set_err(VS_ERR_INVALID, "Unknown metric code %u", m);
    if (dd == 0) return set_err(VS_ERR_INVALID, "bad FAISDART header: d=0");
    *d = dd;
    *metric = (int)m;
    *ntotal = nt;
    *trained = tr != 0;
    return VS_OK;
}

int load_flat(int device, BlobReader &r, int storage, vs_index **out, int *is_trained) {
    int64_t d = 0, ntotal = 0;
    int metric = 0, trained = 0;
    if (int rc = parse_flat_header(r, &d, &metric, &ntotal, &trained)) return rc;
    if (ntotal > (int64_t)INT32_MAX)
        return set_err(VS_ERR_INVALID, "ids are int32: ntotal %lld too large", (long long)ntotal);
    vs_index *x = nullptr;
    if (int rc = vs_index_create(device, d, metric, storage, &x)) return rc;
    struct Owner {
        vs_index *x;
        ~Owner() {
            if (x) vs_index_destroy(x);
        }
    } own{x};
    if (ntotal > 0) {
        if (int rc = vs_index_reserve(x, ntotal)) return rc;
        // the payload goes through one pinned staging buffer of <= 64 MiB
        const int64_t rowb = d * 4;
        const int64_t per = std::max<int64_t>(1, std::min<int64_t>(ntotal, (int64_t)(64 << 20) / rowb));
        HostBuf hb;
        struct Rel {
            HostBuf *h;
            ~Rel() { h->release(); }
        } rel{&hb};
        {
            DeviceGuard g(device);
            VS_HIP(hb.ensure((size_t)per * rowb), "pinned staging");
        }
        for (int64_t r0 = 0; r0 < ntotal; r0 += per) {
            const int64_t m = std::min(per, ntotal - r0);
            if (!r.read(hb.p, m * rowb))
                return set_err(VS_ERR_INVALID, "truncated payload: rows from %lld of %lld missing",
                               (long long)r0, (long long)ntotal);
            if (int rc = vs_index_add(x, hb.p, VS_DTYPE_F32, m)) return rc;
        }
    }
    if (is_trained) *is_trained = trained;
    *out = x;
    own.x = nullptr;
    return VS_OK;
}

}  // namespace

extern "C" {

int vs_index_load_flat(int device, const char *path, int storage, vs_index **out,
                       int *is_trained) {
    if (!out) return set_err(VS_ERR_INVALID, "null output handle");
    *out = nullptr;
    if (!path) return set_err(VS_ERR_INVALID, "null path");
    BlobReader r;
    r.f = fopen(path, "rb");
    if (!r.f) return set_err(VS_ERR_INVALID, "cannot open %s", path);
    return load_flat(device, r, storage, out, is_trained);
}

int vs_index_load_flat_buffer(int device, const void *buf, int64_t len, int storage,
                              vs_index **out, int *is_trained) {
    if (!out) return set_err(VS_ERR_INVALID, "null output handle");
    *out = nullptr;
    if (!buf || len < 0) return set_err(VS_ERR_INVALID, "null or negative-length buffer");
    BlobReader r;
    r.buf = (const unsigned char *)buf;
    r.len = len;
    return load_flat(device, r, storage, out, is_trained);
}

// ---- bench / test support ----

int vs_dev_alloc(int device, int64_t bytes, void **out) {
    if (!out || bytes < 0) return set_err(VS_ERR_INVALID, "bad arguments");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    VS_HIP(hipMalloc(out, (size_t)std::max<int64_t>(bytes, 1)), "hipMalloc");
    return VS_OK;
}

int vs_dev_free(int device, void *p) {
    DeviceGuard g(device);
    if (p) VS_HIP(hipFree(p), "hipFree");
    return VS_OK;
}

int vs_dev_upload(int device, void *dst, const void *src, int64_t bytes) {
    DeviceGuard g(device);
    VS_HIP(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice), "upload");
    return VS_OK;
}

int vs_dev_copy(int device, void *dst, const void *src, int64_t bytes) {
    if (!dst || !src || bytes < 0 || bytes % 16 || ((uintptr_t)dst | (uintptr_t)src) % 16)
        return set_err(VS_ERR_INVALID, "vs_dev_copy: 16-byte aligned buffers and sizes only");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    VS_HIP(vs::launch_copy16(src, dst, bytes / 16, nullptr), "copy kernel");
    VS_HIP(hipDeviceSynchronize(), "copy kernel");
    return VS_OK;
}

int vs_dev_probe(int device, int what, int64_t bytes, double *result) {
    if (!result || what < 0 || what > 2 || (what == 0 && (bytes < (1 << 20) || bytes % 16)))
        return set_err(VS_ERR_INVALID,
                       "vs_dev_probe: what 0 (bytes >= 1 MiB, 16-byte multiple), 1 or 2");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    void *buf = nullptr;
    VS_HIP(hipMalloc(&buf, what == 0 ? (size_t)bytes + 256 : 256), "probe buffer");
    struct Free {
        void *p;
        ~Free() { (void)hipFree(p); }
    } fr{buf};
    hipEvent_t a, b;
    VS_HIP(hipEventCreate(&a), "event");
    VS_HIP(hipEventCreate(&b), "event");
    struct Ev {
        hipEvent_t a, b;
        ~Ev() {
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
        }
    } ev{a, b};
    int num_cu = 256;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) == hipSuccess) num_cu = p.multiProcessorCount;
    const int iters = 4096, blocks = num_cu * 8;
    if (what == 0) VS_HIP(hipMemset(buf, 1, (size_t)bytes), "probe fill");
    double best = 0.0;
    for (int rep = 0; rep < 6; ++rep) {
        VS_HIP(hipEventRecord(a, nullptr), "event");
        if (what == 0)
            VS_HIP(vs::launch_read16(buf, bytes / 16, (uint32_t *)((char *)buf + bytes), nullptr),
                   "read probe");
        else
            VS_HIP(vs::launch_mfma_peak(blocks, iters, what == 2, (float *)buf, nullptr),
                   "mfma probe");
        VS_HIP(hipEventRecord(b, nullptr), "event");
        VS_HIP(hipEventSynchronize(b), "probe");
        float ms = 0.f;
        VS_HIP(hipEventElapsedTime(&ms, a, b), "probe");
        const double v = what == 0 ? (double)bytes / (ms * 1e-3) / 1e9
                                   : (double)blocks * 4 * iters * 8 * 32768.0 / (ms * 1e-3) / 1e12;
        if (rep > 0) best = std::max(best, v);  // the first run warms up
    }
    *result = best;
    return VS_OK;
}

int vs_dev_mfma_chain(int device, int shape, int64_t nsteps, int64_t npass, const uint16_t *A,
                      const uint16_t *B, const float *C, float *D) {
    if (shape < 0 || shape > 1 || nsteps < 1 || nsteps > 4096 || npass < 1 || npass > 4 || !A ||
        !B || !C || !D)
        return set_err(VS_ERR_INVALID,
                       "vs_dev_mfma_chain: shape 0 or 1, 1 <= nsteps <= 4096, 1 <= npass <= 4");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    const size_t mn = shape == 0 ? 32 : 16, K = (size_t)nsteps * (shape == 0 ? 16 : 32);
    const size_t ab = (size_t)npass * mn * K * 2, cb = mn * mn * 4;
    char *buf = nullptr;
    VS_HIP(hipMalloc((void **)&buf, 2 * ab + 2 * cb), "mfma chain buffers");
    struct Free {
        void *p;
        ~Free() { (void)hipFree(p); }
    } fr{buf};
    uint16_t *dA = (uint16_t *)buf, *dB = (uint16_t *)(buf + ab);
    float *dC = (float *)(buf + 2 * ab), *dD = (float *)(buf + 2 * ab + cb);
    VS_HIP(hipMemcpy(dA, A, ab, hipMemcpyHostToDevice), "mfma chain upload");
    VS_HIP(hipMemcpy(dB, B, ab, hipMemcpyHostToDevice), "mfma chain upload");
    VS_HIP(hipMemcpy(dC, C, cb, hipMemcpyHostToDevice), "mfma chain upload");
    VS_HIP(vs::launch_mfma_chain(shape, (int)nsteps, (int)npass, dA, dB, dC, dD, nullptr),
           "mfma chain");
    VS_HIP(hipMemcpy(D, dD, cb, hipMemcpyDeviceToHost), "mfma chain download");
    return VS_OK;
}

int vs_dev_download(int device, void *dst, const void *src, int64_t bytes) {
    DeviceGuard g(device);
    VS_HIP(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost), "download");
    return VS_OK;
}

int vs_gen_normal(int device, void *dst, int out_dtype, int64_t n, int64_t d, uint64_t seed,
                  uint64_t stream, int normalize) {
    if (int rc = check_dtype(out_dtype)) return rc;
    if (n < 0 || d <= 0 || (n > 0 && !dst)) return set_err(VS_ERR_INVALID, "bad arguments");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_err(g.err, "hipSetDevice");
    VS_HIP(vs::launch_gen_normal(dst, out_dtype, n, d, seed, stream, normalize, nullptr),
           "generator");
    VS_HIP(hipDeviceSynchronize(), "generator");
    return VS_OK;
}

int vs_prof_enable(vs_index *x, int on) {
    if (int rc = check_index(x)) return rc;
    x->prof_on = on != 0;
    return VS_OK;
}

int vs_prof_get(vs_index *x, const char *family, int64_t *launches, double *total_ms) {
    if (int rc = check_index(x)) return rc;
    if (!family) return set_err(VS_ERR_INVALID, "null family");
    DeviceGuard g(x->device);
    prof_collect(x);
    auto it = x->prof.find(family);
    if (launches) *launches = it == x->prof.end() ? 0 : it->second.launches;
    if (total_ms) *total_ms = it == x->prof.end() ? 0.0 : it->second.total_ms;
    return VS_OK;
}

int vs_prof_reset(vs_index *x) {
    if (int rc = check_index(x)) return rc;
    DeviceGuard g(x->device);
    prof_collect(x);
    x->prof.clear();
    return VS_OK;
}

int vs_index_sync(vs_index *x) {
    if (int rc = check_index(x)) return rc;
    DeviceGuard g(x->device);
    VS_HIP(hipStreamSynchronize(x->st), "sync");
    return VS_OK;
}

int vs_index_set_option(vs_index *x, const char *name, int64_t value) {
    if (int rc = check_index(x)) return rc;
    if (!name) return set_err(VS_ERR_INVALID, "null option name");
    struct Opt {
        const char *name;
        int VsOptions::*field;
        int lo, hi;
    };
    static const Opt opts[] = {
        {"gemm", &VsOptions::gemm, -1, 1},
        {"gemm_min_nq", &VsOptions::gemm_min_nq, 0, 1 << 30},
        {"gemm_wq", &VsOptions::gemm_wq, 0, 8},
        {"gemm_qb", &VsOptions::gemm_qb, 0, 8},
        {"gemm_kc", &VsOptions::gemm_kc, 0, 64},
        {"gemm4", &VsOptions::gemm4, 0, 1},
        {"share", &VsOptions::share, -1, 1},
        {"coarse", &VsOptions::coarse, 0, 1},
        {"copy16", &VsOptions::copy16, 0, 1},
        {"guess", &VsOptions::guess, 0, 1},
        {"prepass", &VsOptions::prepass, 0, 1},
        {"prepass_log2", &VsOptions::prepass_log2, 10, 20},
        {"scan_kkw", &VsOptions::scan_kkw, 0, 4096},
        {"scan_nw8", &VsOptions::scan_nw8, 0, 1},
        {"km16", &VsOptions::km16, 0, 1},
        {"km16_rt", &VsOptions::km16_rt, 2, 4},
        {"km16_nqb", &VsOptions::km16_nqb, 2, 4},
        {"pick_order", &VsOptions::pick_order, 0, 1},
        {"merge_mu", &VsOptions::merge_mu, 0, 8},
        {"merge_g", &VsOptions::merge_g, 0, 64},
        {"guess_div_log2", &VsOptions::guess_div_log2, 0, 10},
        {"kmin_init", &VsOptions::kmin_init, 0, 1},
        {"assign_order", &VsOptions::assign_order, 0, 1},
    };
    if (strcmp(name, "fail_alloc") == 0) {  // not a planner option: this thread's countdown
        if (value < 0) return set_err(VS_ERR_INVALID, "option fail_alloc: value %lld < 0", (long long)value);
        g_fail_alloc = value;
        return VS_OK;
    }
    for (const Opt &o : opts) {
        if (strcmp(o.name, name) != 0) continue;
        const bool hole = (o.field == &VsOptions::km16_rt && value == 3) ||
                          (o.field == &VsOptions::km16_nqb && value == 3) ||
                          (o.field == &VsOptions::merge_mu && value > 2 && value != 4 && value != 8);
        if (value < o.lo || value > o.hi || hole)
            return set_err(VS_ERR_INVALID, "option %s: value %lld outside [%d, %d]", name,
                           (long long)value, o.lo, o.hi);
        x->opt.*(o.field) = (int)value;
        return VS_OK;
    }
    return set_err(VS_ERR_INVALID, "unknown option \"%s\"", name);
}

}  // extern "C"
