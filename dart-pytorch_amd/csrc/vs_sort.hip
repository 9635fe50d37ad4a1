// vs_sort.hip -- stable key sort used by the k-means update (grouping point
// ids by cluster in increasing point order).  rocPRIM's radix sort is stable.
#include <cstring>
#include <rocprim/device/device_radix_sort.hpp>

#include "vs_internal.h"

namespace vs {

hipError_t sort_pairs_by_key(void *tmp, size_t &tmp_bytes, const int32_t *kin, int32_t *kout,
                             const int32_t *vin, int32_t *vout, int64_t n, int key_bits,
                             hipStream_t st) {
    return rocprim::radix_sort_pairs(tmp, tmp_bytes, kin, kout, vin, vout, (size_t)n, 0, key_bits,
                                     st);
}

}  // namespace vs
