// scan_sort.h -- device-wide prefix sums and stable radix sort (scan_sort.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace annc {

// Scratch bytes of the prefix sums over n values.
size_t scan_temp_bytes(int64_t n);
// out[i] = sum of in[0..i) (exclusive) or in[0..i] (inclusive), n < 2^31;
// in and out do not overlap.  temp: scan_temp_bytes(n) bytes of device
// memory.
int exclusive_sum(hipStream_t s, const int32_t* in, int32_t* out, int64_t n, void* temp);
int inclusive_sum(hipStream_t s, const int32_t* in, int32_t* out, int64_t n, void* temp);

// Scratch bytes of radix_sort_pairs over n pairs.
size_t radix_sort_temp_bytes(int64_t n);
// Stable sort of n (key, value) pairs by the low end_bit bits of the key,
// 8 bits per pass, ping-ponging between *keys/*vals and *keys_alt/*vals_alt;
// on return *keys and *vals point at the sorted pairs (the pointers are
// swapped once per pass).  temp: radix_sort_temp_bytes(n) bytes.
int radix_sort_pairs(hipStream_t s, uint32_t** keys, uint32_t** keys_alt, int32_t** vals,
                     int32_t** vals_alt, int64_t n, int end_bit, void* temp);

}  // namespace annc
