// Device-wide sort, scan and reduction primitives of the preparation paths (border
// selection, categorical columns), over rocPRIM's native device API.  Each wrapper keeps the
// two-phase temporary-storage protocol: a call with tmp == nullptr only sets bytes.
#pragma once
#include <hip/hip_runtime.h>

#include <cstring>
#include <limits>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_reduce.hpp>
#include <rocprim/device/device_scan.hpp>
#include <rocprim/device/device_segmented_radix_sort.hpp>

namespace cbh {
namespace prim {

// Stable LSD radix sort of (key, value) pairs on key bits [bb, eb).
template <class K, class V>
hipError_t sort_pairs(void* tmp, size_t& bytes, const K* kin, K* kout, const V* vin, V* vout, int n, int bb, int eb,
                      hipStream_t st = 0) {
    return rocprim::radix_sort_pairs(tmp, bytes, kin, kout, vin, vout, (unsigned int)n, (unsigned int)bb,
                                     (unsigned int)eb, st);
}

// Radix sort of the keys of every segment [beg[s], end[s]) independently.
template <class K>
hipError_t segmented_sort_keys(void* tmp, size_t& bytes, const K* kin, K* kout, int n, int segs, const int* beg,
                               const int* end, int bb, int eb, hipStream_t st = 0) {
    return rocprim::segmented_radix_sort_keys(tmp, bytes, kin, kout, (unsigned int)n, (unsigned int)segs, beg, end,
                                              (unsigned int)bb, (unsigned int)eb, st);
}

template <class T>
hipError_t exclusive_sum(void* tmp, size_t& bytes, const T* in, T* out, int n, hipStream_t st = 0) {
    return rocprim::exclusive_scan(tmp, bytes, in, out, T(0), (size_t)n, rocprim::plus<T>(), st);
}

template <class T>
hipError_t inclusive_sum(void* tmp, size_t& bytes, const T* in, T* out, int n, hipStream_t st = 0) {
    return rocprim::inclusive_scan(tmp, bytes, in, out, (size_t)n, rocprim::plus<T>(), st);
}

template <class T>
hipError_t inclusive_max(void* tmp, size_t& bytes, const T* in, T* out, int n, hipStream_t st = 0) {
    return rocprim::inclusive_scan(tmp, bytes, in, out, (size_t)n, rocprim::maximum<T>(), st);
}

// out[0] = max of in[0, n) (n >= 1).
template <class T>
hipError_t reduce_max(void* tmp, size_t& bytes, const T* in, T* out, int n, hipStream_t st = 0) {
    return rocprim::reduce(tmp, bytes, in, out, std::numeric_limits<T>::lowest(), (size_t)n, rocprim::maximum<T>(),
                           st);
}

}  // namespace prim
}  // namespace cbh
