// vs_sort.hip -- the sorting paths of libvs_hip.so (rocPRIM radix sorts):
//   - the stable key sort of the k-means update (point ids grouped by
//     cluster in increasing point order);
//   - exact top-k for any k: every row's fp64 score as a 64-bit key
//     (order-preserving code of the fp32 key, then the id), sorted per query.
#include <cstring>
#include <rocprim/device/device_radix_sort.hpp>

#include "vs_device.h"

namespace vs {

hipError_t sort_pairs_by_key(void *tmp, size_t &tmp_bytes, const int32_t *kin, int32_t *kout,
                             const int32_t *vin, int32_t *vout, int64_t n, int key_bits,
                             hipStream_t st) {
    return rocprim::radix_sort_pairs(tmp, tmp_bytes, kin, kout, vin, vout, (size_t)n, 0, key_bits,
                                     st);
}

// keys[qi][r] = enc_order(key) << 32 | r, key = fp32 score (L2) or -fp32
// score (IP) of query qi and row r, the score in the reference's fp64
// arithmetic (index_flat.dart:75-90).  One thread per row; the chunk's
// queries are staged QG at a time in LDS, zero past d (exact_score reads
// whole 64-element batches).
__global__ __launch_bounds__(256) void exact_keys_kernel(const void *xb, int storage, int64_t ld,
                                                         int64_t d, int metric, const float *qf,
                                                         int64_t nqc, int64_t n, int qg_max,
                                                         uint64_t *keys) {
    extern __shared__ __align__(16) char smem[];
    float *qs = (float *)smem;  // [qg_max][ld]
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (int64_t q0 = 0; q0 < nqc; q0 += qg_max) {
        const int64_t qn = min((int64_t)qg_max, nqc - q0);
        __syncthreads();
        for (int64_t t = threadIdx.x; t < qn * ld; t += 256) {
            const int64_t qi = t / ld, j = t % ld;
            qs[t] = j < d ? qf[(q0 + qi) * d + j] : 0.0f;
        }
        __syncthreads();
        if (r < n) {
            for (int64_t qi = 0; qi < qn; ++qi) {
                const double ex = storage == 1 ? exact_score<1>(qs + qi * ld, xb, ld, r, d, metric)
                                               : exact_score<0>(qs + qi * ld, xb, ld, r, d, metric);
                const float key = metric == 0 ? (float)ex : -(float)ex;
                keys[(q0 + qi) * n + r] = ((uint64_t)enc_order(key) << 32) | (uint32_t)r;
            }
        }
    }
}

// D / I [k] of one query from its sorted keys (sentinels past n).
__global__ void extract_topk_kernel(const uint64_t *__restrict__ sorted, int64_t n, int64_t k,
                                    int metric, float *__restrict__ D, int32_t *__restrict__ I) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= k) return;
    if (t < n) {
        const uint64_t w = sorted[t];
        const float key = dec_order((uint32_t)(w >> 32));
        D[t] = metric == 0 ? key : -key;
        I[t] = (int32_t)(uint32_t)w;
    } else {
        D[t] = metric == 0 ? VS_INF : -VS_INF;
        I[t] = -1;
    }
}

hipError_t exact_sort_topk(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                           const float *qf, int64_t nq, int64_t n, int64_t k, float *D, int32_t *I,
                           uint64_t *keys, int64_t qchunk, void *tmp, size_t &tmp_bytes,
                           hipStream_t st) {
    if (n <= 0 || n > (int64_t)UINT32_MAX) return hipErrorInvalidValue;
    if (!tmp) {
        return rocprim::radix_sort_keys(nullptr, tmp_bytes, (const uint64_t *)nullptr,
                                        (uint64_t *)nullptr, (size_t)n, 0, 64, st);
    }
    if (nq <= 0 || qchunk <= 0) return hipSuccess;
    const int qg_max = (int)std::max<int64_t>(1, std::min<int64_t>(16, 32768 / (ld * 4)));
    const size_t lds = (size_t)qg_max * ld * 4;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)exact_keys_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    uint64_t *out = keys + qchunk * n;
    for (int64_t q0 = 0; q0 < nq; q0 += qchunk) {
        const int64_t nqc = std::min(qchunk, nq - q0);
        exact_keys_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), lds, st>>>(
            xb, storage, ld, d, metric, qf + q0 * d, nqc, n, qg_max, keys);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        for (int64_t qi = 0; qi < nqc; ++qi) {
            size_t tb = tmp_bytes;
            e = rocprim::radix_sort_keys(tmp, tb, keys + qi * n, out, (size_t)n, 0, 64, st);
            if (e != hipSuccess) return e;
            extract_topk_kernel<<<dim3((unsigned)((k + 255) / 256)), dim3(256), 0, st>>>(
                out, n, k, metric, D + (q0 + qi) * k, I + (q0 + qi) * k);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// keys[p] = enc_order(key) << 32 | ids[p] for one query (fp32 row qf [d])
// against the rows ids[0 .. m): the exact_keys_kernel arithmetic over a
// given row subset.  One thread per candidate; the query staged in LDS,
// zero past d.
__global__ __launch_bounds__(256) void exact_keys_ids_kernel(const void *xb, int storage,
                                                             int64_t ld, int64_t d, int metric,
                                                             const float *qf, const int32_t *ids,
                                                             int64_t m, uint64_t *keys) {
    extern __shared__ __align__(16) char smem[];
    float *qs = (float *)smem;  // [ld]
    for (int64_t j = threadIdx.x; j < ld; j += 256) qs[j] = j < d ? qf[j] : 0.0f;
    __syncthreads();
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= m) return;
    const int64_t id = ids[p];
    const double ex = storage == 1 ? exact_score<1>(qs, xb, ld, id, d, metric)
                                   : exact_score<0>(qs, xb, ld, id, d, metric);
    const float key = metric == 0 ? (float)ex : -(float)ex;
    keys[p] = ((uint64_t)enc_order(key) << 32) | (uint32_t)id;
}

hipError_t exact_sort_topk_ids(const void *xb, int storage, int64_t ld, int64_t d, int metric,
                               const float *qf, const int32_t *ids, int64_t m, int64_t k, float *D,
                               int32_t *I, uint64_t *keys, void *tmp, size_t &tmp_bytes,
                               hipStream_t st) {
    if (m < 0 || m > (int64_t)UINT32_MAX) return hipErrorInvalidValue;
    if (!tmp) {
        return rocprim::radix_sort_keys(nullptr, tmp_bytes, (const uint64_t *)nullptr,
                                        (uint64_t *)nullptr, (size_t)std::max<int64_t>(m, 1), 0,
                                        64, st);
    }
    uint64_t *out = keys + m;
    if (m > 0) {
        const size_t lds = (size_t)ld * 4;
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute((const void *)exact_keys_ids_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        exact_keys_ids_kernel<<<dim3((unsigned)((m + 255) / 256)), dim3(256), lds, st>>>(
            xb, storage, ld, d, metric, qf, ids, m, keys);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        size_t tb = tmp_bytes;
        e = rocprim::radix_sort_keys(tmp, tb, keys, out, (size_t)m, 0, 64, st);
        if (e != hipSuccess) return e;
    }
    extract_topk_kernel<<<dim3((unsigned)((k + 255) / 256)), dim3(256), 0, st>>>(out, m, k, metric,
                                                                              D, I);
    return hipGetLastError();
}

}  // namespace vs
