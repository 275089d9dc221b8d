// gather.hip -- unique + gather (KPFusedGather) on gfx950.
//
// Reference: annc/tensorflow/kernels/embedding_fused_gather.cc:26-85.  The
// keys of one column are de-duplicated in order of first occurrence (an
// unordered_map walk over the rows), every row gets the index of its key in
// that order, and the table rows of the unique keys are copied out.
//
// Device formulation (the outputs do not depend on thread timing):
//   1. every key goes into an open-addressing hash table (64-bit CAS on the
//      key, linear probing, capacity a power of two >= 2n, a separate slot
//      for the empty marker's own value) and the slot keeps the smallest
//      position of its key (atomicMin): the key's first occurrence;
//   2. position i is a first occurrence iff its slot's minimum is i; an
//      inclusive scan of those marks numbers the unique keys in order of
//      first occurrence (the reference's order), U = the last sum;
//   3. indices[i] = number of the first occurrence of i's key; that
//      occurrence also writes unique[number] = key;
//   4. out rows of the U unique keys, G lanes per row, 16-byte loads where
//      the rows allow.
// U is only known on the device; kernels sized by n test r < U themselves.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <climits>

#include "common.h"
#include "embedding_impl.h"

namespace annc {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kEmpty = INT64_MIN;  // key of an unused slot

// MurmurHash3's 64-bit finaliser (fmix64): spreads nearby keys over the table.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return x;
}

__global__ void ug_clear_kernel(int64_t* __restrict__ tab_key, int32_t* __restrict__ tab_first,
                                int64_t slots) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= slots) return;
  tab_key[c] = kEmpty;
  tab_first[c] = INT_MAX;
}

// Probe for `key` from its hash, inserting it into a free slot if it is
// new; returns the slot, or -1 after `cap` probes (cannot happen while at
// most cap/2 distinct keys are inserted).  A slot's key never changes once
// set, so a plain read that already shows a key decides without an atomic.
__device__ __forceinline__ int64_t probe_insert(int64_t* tab_key, int64_t cap, int64_t key) {
  int64_t h = static_cast<int64_t>(mix64(static_cast<uint64_t>(key)) & (uint64_t)(cap - 1));
  for (int64_t probe = 0; probe < cap; ++probe) {
    int64_t seen = __hip_atomic_load(tab_key + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (seen == kEmpty)
      seen = static_cast<int64_t>(atomicCAS(reinterpret_cast<unsigned long long*>(tab_key + h),
                                            static_cast<unsigned long long>(kEmpty),
                                            static_cast<unsigned long long>(key)));
    if (seen == kEmpty || seen == key) return h;
    h = (h + 1) & (cap - 1);
  }
  return -1;
}

// Insert workgroups of 1024 threads over 2048 positions: a key that is
// frequent in the data costs one global atomic per 2048 positions, not per
// 256 (configs[2]'s ids: 42.5 -> 37.4 us for the whole unique + gather;
// 4096 positions, at half the workgroups, was slower again).
constexpr int kUgThreads = 1024;         // threads of an insert workgroup
constexpr int kUgBlock = 2048;           // positions per workgroup
constexpr int kUgLocal = 2 * kUgBlock;   // LDS table slots (+1 for the empty marker's value)

// Slot of every position's key in the global table, whose slots keep their
// key's smallest position.  Each workgroup first de-duplicates its 256
// positions in an LDS table (block minimum per key), then inserts each of
// its distinct keys once: a key that is frequent in the data costs one
// global CAS and one atomicMin per workgroup, not one per occurrence.
__global__ __launch_bounds__(kUgThreads) void ug_insert_kernel(
    const int64_t* __restrict__ keys, int64_t stride, int64_t n, int64_t cap,
    int64_t* __restrict__ tab_key, int32_t* __restrict__ tab_first,
    int32_t* __restrict__ slot_of, int* __restrict__ status) {
  __shared__ int64_t lkey[kUgLocal];
  __shared__ int32_t lfirst[kUgLocal + 1];
  __shared__ int32_t lslot[kUgLocal + 1];
  __shared__ int lempty;  // some position holds the empty marker's value
  constexpr int kPer = kUgBlock / kUgThreads;
  for (int l = threadIdx.x; l < kUgLocal; l += kUgThreads) lkey[l] = kEmpty;
  for (int l = threadIdx.x; l <= kUgLocal; l += kUgThreads) lfirst[l] = INT_MAX;
  if (threadIdx.x == 0) lempty = 0;
  __syncthreads();
  const int64_t b0 = (int64_t)blockIdx.x * kUgBlock;
  int local[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t i = b0 + u * kUgThreads + threadIdx.x;
    local[u] = -1;
    if (i >= n) continue;
    const int64_t key = keys[i * stride];
    int l = kUgLocal;
    if (key == kEmpty) {
      lempty = 1;
    } else {
      int h = static_cast<int>(mix64(static_cast<uint64_t>(key)) & (kUgLocal - 1));
      for (int probe = 0; probe < kUgLocal; ++probe) {  // <= kUgBlock keys in 2x slots
        const int64_t seen = static_cast<int64_t>(atomicCAS(
            reinterpret_cast<unsigned long long*>(lkey + h), static_cast<unsigned long long>(kEmpty),
            static_cast<unsigned long long>(key)));
        if (seen == kEmpty || seen == key) break;
        h = (h + 1) & (kUgLocal - 1);
      }
      l = h;
    }
    atomicMin(lfirst + l, static_cast<int32_t>(i));
    local[u] = l;
  }
  __syncthreads();
  for (int l = threadIdx.x; l <= kUgLocal; l += kUgThreads) {
    const bool used = l < kUgLocal ? lkey[l] != kEmpty : lempty != 0;
    if (!used) continue;
    int64_t g = cap;  // the empty marker's value has the extra global slot
    if (l < kUgLocal) {
      g = probe_insert(tab_key, cap, lkey[l]);
      if (g < 0) {  // reported, never hangs
        atomicOr(status, 2);
        g = cap;
      }
    }
    const int32_t first = lfirst[l];
    if (__hip_atomic_load(tab_first + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) > first)
      atomicMin(tab_first + g, first);
    lslot[l] = static_cast<int32_t>(g);
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t i = b0 + u * kUgThreads + threadIdx.x;
    if (i < n) slot_of[i] = lslot[local[u]];
  }
}

__global__ void ug_mark_kernel(const int32_t* __restrict__ slot_of,
                               const int32_t* __restrict__ tab_first, int64_t n,
                               int32_t* __restrict__ first_mark) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  first_mark[i] = tab_first[slot_of[i]] == static_cast<int32_t>(i) ? 1 : 0;
}

// number[i] = inclusive count of first occurrences up to i
__global__ void ug_output_kernel(const int64_t* __restrict__ keys, int64_t stride, int64_t n,
                                 const int32_t* __restrict__ slot_of,
                                 const int32_t* __restrict__ tab_first,
                                 const int32_t* __restrict__ number, int32_t* __restrict__ indices,
                                 int64_t* __restrict__ unique, int64_t* __restrict__ num_unique) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int32_t first = tab_first[slot_of[i]];
  const int32_t r = number[first] - 1;
  indices[i] = r;
  if (first == static_cast<int32_t>(i)) unique[r] = keys[i * stride];
  if (i == n - 1) num_unique[0] = number[n - 1];
}

// out[r, :] = table[unique[r], :] for r < U, G lanes per row (VEC floats per
// lane); keys outside the table give a zero row and set the status word.
template <int G, int VEC>
__global__ __launch_bounds__(kThreads) void ug_gather_kernel(
    const float* __restrict__ table, int64_t rows, int64_t dim, const int64_t* __restrict__ unique,
    const int64_t* __restrict__ num_unique, int64_t n, float* __restrict__ out,
    int* __restrict__ status) {
  const int g = threadIdx.x & (G - 1);
  const int64_t r = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / G;
  if (r >= n || r >= num_unique[0]) return;
  const int64_t id = unique[r];
  const bool ok = id >= 0 && id < rows;
  if (!ok && g == 0) atomicOr(status, 1);
  const float* src = table + (ok ? id : 0) * dim;
  float* dst = out + r * dim;
  for (int64_t c = (int64_t)g * VEC; c < dim; c += (int64_t)G * VEC) {
    if constexpr (VEC == 4) {
      typedef float V __attribute__((ext_vector_type(4)));
      const V v = ok ? *reinterpret_cast<const V*>(src + c) : V(0.0f);
      *reinterpret_cast<V*>(dst + c) = v;
    } else {
      dst[c] = ok ? src[c] : 0.0f;
    }
  }
}

__global__ void store_i64_kernel(int64_t* p, int64_t v) { *p = v; }

template <int VEC>
void launch_ug_gather(hipStream_t s, int g, const float* table, int64_t rows, int64_t dim,
                      const int64_t* unique, const int64_t* num_unique, int64_t n, float* out,
                      int* status) {
  const dim3 grid((unsigned)ceil_div(n * g, kThreads));
  switch (g) {
#define ANNC_UG(G)                                                                          \
  case G:                                                                                   \
    hipLaunchKernelGGL((ug_gather_kernel<G, VEC>), grid, dim3(kThreads), 0, s, table, rows, \
                       dim, unique, num_unique, n, out, status);                            \
    break;
    ANNC_UG(1) ANNC_UG(2) ANNC_UG(4) ANNC_UG(8) ANNC_UG(16) ANNC_UG(32) ANNC_UG(64)
#undef ANNC_UG
  }
}

// ---------------------------------------------------------------------------
// First occurrences over a small key range (keys in [kmin, kmin + range)):
// first[key - kmin] is indexed directly instead of through the hash table.
// ---------------------------------------------------------------------------
__global__ void fo_fill_kernel(int32_t* __restrict__ first, int64_t range) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c < range) first[c] = INT_MAX;
}

// first[key - kmin] = smallest position of the key; a plain read that already
// shows a smaller position skips the atomic (frequent keys cost one atomic
// per few workgroups, not one per occurrence)
__global__ void fo_min_kernel(const int64_t* __restrict__ keys, int64_t stride, int64_t n,
                              int64_t kmin, int32_t* __restrict__ first) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  int32_t* f = first + (keys[i * stride] - kmin);
  if (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) > static_cast<int32_t>(i))
    atomicMin(f, static_cast<int32_t>(i));
}

__global__ void fo_mark_kernel(const int64_t* __restrict__ keys, int64_t stride, int64_t n,
                               int64_t kmin, const int32_t* __restrict__ first,
                               int32_t* __restrict__ first_mark) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  first_mark[i] = first[keys[i * stride] - kmin] == static_cast<int32_t>(i) ? 1 : 0;
}

// Without global atomics, for small ranges (the segment column of
// KPFusedSparseSegmentReduceNonzero): workgroup b takes positions
// [b*kFoBlock, (b+1)*kFoBlock), keeps each key's smallest position in an
// LDS table (LDS atomics) and writes the table to part[b][0, range);
// fo_merge_kernel then takes the minimum over the workgroups.  The global
// table of a small range is a few cache lines, which serialise the atomics
// of every position on them.
constexpr int kFoThreads = 1024;
constexpr int kFoItems = 4;
constexpr int kFoBlock = kFoThreads * kFoItems;  // positions per workgroup
constexpr int64_t kFoLdsRange = 8192;            // keys in LDS (32 KiB)
constexpr int64_t kFoMaxBlocks = 64;             // workgroups merged per key

__global__ __launch_bounds__(kFoThreads) void fo_local_min_kernel(
    const int64_t* __restrict__ keys, int64_t stride, int64_t n, int64_t kmin, int range,
    int32_t* __restrict__ part) {
  extern __shared__ int32_t fo_tab[];
  for (int r = threadIdx.x; r < range; r += kFoThreads) fo_tab[r] = INT_MAX;
  const int64_t b0 = (int64_t)blockIdx.x * kFoBlock;
  int64_t k[kFoItems];
#pragma unroll
  for (int u = 0; u < kFoItems; ++u) {  // loads issued together (position clamped)
    const int64_t i = b0 + u * kFoThreads + threadIdx.x;
    k[u] = keys[(i < n ? i : n - 1) * stride];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kFoItems; ++u) {
    const int64_t i = b0 + u * kFoThreads + threadIdx.x;
    if (i < n) atomicMin(fo_tab + (k[u] - kmin), static_cast<int32_t>(i));
  }
  __syncthreads();
  int32_t* dst = part + (int64_t)blockIdx.x * range;
  for (int r = threadIdx.x; r < range; r += kFoThreads) dst[r] = fo_tab[r];
}

__global__ void fo_merge_kernel(const int32_t* __restrict__ part, int nblk, int range,
                                int32_t* __restrict__ first) {
  const int r = blockIdx.x * kThreads + threadIdx.x;
  if (r >= range) return;
  int32_t m = INT_MAX;
  for (int b = 0; b < nblk; ++b) m = min(m, part[(int64_t)b * range + r]);
  first[r] = m;
}

// number[i] = inclusive count of first occurrences up to i
__global__ void fo_output_kernel(const int64_t* __restrict__ keys, int64_t stride, int64_t n,
                                 int64_t kmin, const int32_t* __restrict__ first,
                                 const int32_t* __restrict__ number,
                                 int32_t* __restrict__ indices, int64_t* __restrict__ unique,
                                 int64_t* __restrict__ num_unique) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t key = keys[i * stride];
  const int32_t f = first[key - kmin];
  const int32_t r = number[f] - 1;
  indices[i] = r;
  if (f == static_cast<int32_t>(i)) unique[r] = key;
  if (i == n - 1) num_unique[0] = number[n - 1];
}

}  // namespace

int first_occurrence_range(hipStream_t s, const int64_t* keys, int64_t stride, int64_t n,
                           int64_t kmin, int64_t range, int64_t* num_unique, int64_t* unique,
                           int32_t* indices) {
  ANNC_REQUIRE(n > 0 && n < INT_MAX && range >= 1, "bad first-occurrence size");
  size_t scan = 0;
  ANNC_HIP_TRY(hipcub::DeviceScan::InclusiveSum(nullptr, scan, (const int32_t*)nullptr,
                                                (int32_t*)nullptr, (int)n, s));
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const int64_t nblk = ceil_div(n, kFoBlock);
  const bool local = range <= kFoLdsRange && nblk <= kFoMaxBlocks;
  const size_t fb = align(sizeof(int32_t) * (size_t)range);
  const size_t n4 = align(sizeof(int32_t) * (size_t)n);
  const size_t pb = local ? align(sizeof(int32_t) * (size_t)(nblk * range)) : 0;
  char* ws = static_cast<char*>(stream_workspace(s, fb + 2 * n4 + pb + align(scan)));
  if (!ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  int32_t* first = reinterpret_cast<int32_t*>(ws);
  int32_t* mark = reinterpret_cast<int32_t*>(ws + fb);
  int32_t* number = reinterpret_cast<int32_t*>(ws + fb + n4);
  int32_t* part = reinterpret_cast<int32_t*>(ws + fb + 2 * n4);
  void* tmp = ws + fb + 2 * n4 + pb;
  const dim3 grid((unsigned)ceil_div(n, kThreads));
  if (local) {
    hipLaunchKernelGGL(fo_local_min_kernel, dim3((unsigned)nblk), dim3(kFoThreads),
                       sizeof(int32_t) * (size_t)range, s, keys, stride, n, kmin,
                       static_cast<int>(range), part);
    ANNC_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(fo_merge_kernel, dim3((unsigned)ceil_div(range, kThreads)), dim3(kThreads),
                       0, s, part, static_cast<int>(nblk), static_cast<int>(range), first);
    ANNC_HIP_TRY(hipGetLastError());
  } else {
    hipLaunchKernelGGL(fo_fill_kernel, dim3((unsigned)ceil_div(range, kThreads)), dim3(kThreads),
                       0, s, first, range);
    ANNC_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(fo_min_kernel, grid, dim3(kThreads), 0, s, keys, stride, n, kmin, first);
    ANNC_HIP_TRY(hipGetLastError());
  }
  hipLaunchKernelGGL(fo_mark_kernel, grid, dim3(kThreads), 0, s, keys, stride, n, kmin, first,
                     mark);
  ANNC_HIP_TRY(hipGetLastError());
  ANNC_HIP_TRY(hipcub::DeviceScan::InclusiveSum(tmp, scan, mark, number, (int)n, s));
  hipLaunchKernelGGL(fo_output_kernel, grid, dim3(kThreads), 0, s, keys, stride, n, kmin, first,
                     number, indices, unique, num_unique);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

int unique_gather(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                  const int64_t* keys, int64_t stride, int64_t n, int64_t* num_unique,
                  int64_t* unique, int32_t* indices, float* out) {
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  int64_t cap = 1024;
  while (cap < 2 * n) cap <<= 1;
  size_t scan = 0;
  ANNC_HIP_TRY(hipcub::DeviceScan::InclusiveSum(nullptr, scan, (const int32_t*)nullptr,
                                                (int32_t*)nullptr, (int)n, s));
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t kb = align(sizeof(int64_t) * (size_t)(cap + 1));
  const size_t fb = align(sizeof(int32_t) * (size_t)(cap + 1));
  const size_t n4 = align(sizeof(int32_t) * (size_t)n);
  char* ws = static_cast<char*>(stream_workspace(s, kb + fb + 3 * n4 + align(scan)));
  if (!ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  int64_t* tab_key = reinterpret_cast<int64_t*>(ws);
  int32_t* tab_first = reinterpret_cast<int32_t*>(ws + kb);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws + kb + fb);
  int32_t* mark = reinterpret_cast<int32_t*>(ws + kb + fb + n4);
  int32_t* number = reinterpret_cast<int32_t*>(ws + kb + fb + 2 * n4);
  void* tmp = ws + kb + fb + 3 * n4;
  const dim3 grid((unsigned)ceil_div(n, kThreads));
  hipLaunchKernelGGL(ug_clear_kernel, dim3((unsigned)ceil_div(cap + 1, kThreads)), dim3(kThreads),
                     0, s, tab_key, tab_first, cap + 1);
  ANNC_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(ug_insert_kernel, dim3((unsigned)ceil_div(n, kUgBlock)), dim3(kUgThreads), 0, s,
                     keys, stride, n, cap, tab_key, tab_first, slot_of, status);
  ANNC_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(ug_mark_kernel, grid, dim3(kThreads), 0, s, slot_of, tab_first, n, mark);
  ANNC_HIP_TRY(hipGetLastError());
  ANNC_HIP_TRY(hipcub::DeviceScan::InclusiveSum(tmp, scan, mark, number, (int)n, s));
  hipLaunchKernelGGL(ug_output_kernel, grid, dim3(kThreads), 0, s, keys, stride, n, slot_of,
                     tab_first, number, indices, unique, num_unique);
  ANNC_HIP_TRY(hipGetLastError());
  if (dim > 0) {
    int g = 1;
    const bool vec = dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(table) |
                                       reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    const int64_t lanes = vec ? dim / 4 : dim;
    while (g < 64 && g < lanes) g <<= 1;
    if (vec)
      launch_ug_gather<4>(s, g, table, rows, dim, unique, num_unique, n, out, status);
    else
      launch_ug_gather<1>(s, g, table, rows, dim, unique, num_unique, n, out, status);
    ANNC_HIP_TRY(hipGetLastError());
  }
  return ANNC_OK;
}

}  // namespace annc

extern "C" int annc_hip_unique_gather(void* stream, const float* table, int64_t rows, int64_t dim,
                                      const int64_t* keys, int64_t key_stride, int64_t n,
                                      int64_t* num_unique, int64_t* unique, int32_t* indices,
                                      float* out) {
  using namespace annc;
  ANNC_REQUIRE(rows >= 0 && dim >= 0 && n >= 0 && key_stride >= 1, "bad dimensions");
  ANNC_REQUIRE(n < INT_MAX, "too many keys");
  ANNC_REQUIRE(num_unique != nullptr, "null num_unique");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n == 0) {
    hipLaunchKernelGGL(store_i64_kernel, dim3(1), dim3(1), 0, s, num_unique, int64_t(0));
    ANNC_HIP_TRY(hipGetLastError());
    return set_error(ANNC_OK, "");
  }
  ANNC_REQUIRE(keys && unique && indices && (dim == 0 || (table && out)), "null pointer");
  const int rc = unique_gather(s, table, rows, dim, keys, key_stride, n, num_unique, unique,
                               indices, out);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}
