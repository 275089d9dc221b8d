// gather.hip -- unique + gather (KPFusedGather) on gfx950.
//
// Reference: annc/tensorflow/kernels/embedding_fused_gather.cc:26-85.  The
// keys of one column are de-duplicated in order of first occurrence (an
// unordered_map walk over the rows), every row gets the index of its key in
// that order, and the table rows of the unique keys are copied out.
//
// Device formulation (all steps keep the reference's order exactly):
//   1. (key, position) pairs sorted by key with a stable radix sort, so the
//      first element of each run of equal keys is the key's first occurrence;
//   2. run heads flagged and inclusive-summed: run id of every sorted element,
//      U = number of runs;
//   3. the runs sorted by first position (positions of absent runs padded to
//      INT32_MAX so they sort last): rank of a run = its place in that order;
//   4. unique[rank] = key, indices[position] = rank, out_data[rank] = row.
// U is only known on the device; kernels sized by n test r < U themselves.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <climits>

#include "common.h"

namespace annc {
namespace {

constexpr int kThreads = 256;

__global__ void extract_keys_kernel(const int64_t* __restrict__ keys, int64_t stride, int64_t n,
                                    int64_t* __restrict__ k_out, int32_t* __restrict__ pos_out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  k_out[i] = keys[i * stride];
  pos_out[i] = static_cast<int32_t>(i);
}

__global__ void run_heads_kernel(const int64_t* __restrict__ sk, int64_t n,
                                 int32_t* __restrict__ head, int32_t* __restrict__ first_pos) {
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= n) return;
  head[j] = (j == 0 || sk[j] != sk[j - 1]) ? 1 : 0;
  first_pos[j] = INT_MAX;  // padding for runs that do not exist
}

// run = runid[j] - 1 for the head j of every run
__global__ void run_first_kernel(const int64_t* __restrict__ sk, const int32_t* __restrict__ sp,
                                 const int32_t* __restrict__ head,
                                 const int32_t* __restrict__ runid, int64_t n,
                                 int32_t* __restrict__ first_pos, int32_t* __restrict__ run_idx,
                                 int64_t* __restrict__ run_key) {
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= n) return;
  run_idx[j] = static_cast<int32_t>(j);
  if (head[j]) {
    const int32_t r = runid[j] - 1;
    first_pos[r] = sp[j];
    run_key[r] = sk[j];
  }
}

__global__ void rank_kernel(const int32_t* __restrict__ order, const int64_t* __restrict__ run_key,
                            const int32_t* __restrict__ runid, int64_t n,
                            int32_t* __restrict__ rank_of_run, int64_t* __restrict__ unique,
                            int64_t* __restrict__ num_unique) {
  const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int32_t total = runid[n - 1];
  if (r == 0) num_unique[0] = total;
  if (r >= total) return;
  const int32_t run = order[r];
  rank_of_run[run] = static_cast<int32_t>(r);
  unique[r] = run_key[run];
}

__global__ void indices_kernel(const int32_t* __restrict__ sp, const int32_t* __restrict__ runid,
                               const int32_t* __restrict__ rank_of_run, int64_t n,
                               int32_t* __restrict__ indices) {
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= n) return;
  indices[sp[j]] = rank_of_run[runid[j] - 1];
}

// out[r, :] = table[unique[r], :] for r < U; ids outside the table give a
// zero row and set the stream's status word.
__global__ void gather_unique_kernel(const float* __restrict__ table, int64_t rows, int64_t dim,
                                     const int64_t* __restrict__ unique,
                                     const int32_t* __restrict__ runid, int64_t n,
                                     float* __restrict__ out, int* __restrict__ status) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t total = runid[n - 1];
  if (t >= total * dim) return;
  const int64_t r = t / dim, d = t - r * dim;
  const int64_t id = unique[r];
  const bool ok = id >= 0 && id < rows;
  if (!ok && d == 0) atomicOr(status, 1);
  out[t] = ok ? table[id * dim + d] : 0.0f;
}

__global__ void store_i64_kernel(int64_t* p, int64_t v) { *p = v; }

}  // namespace

int unique_gather(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                  const int64_t* keys, int64_t stride, int64_t n, int64_t* num_unique,
                  int64_t* unique, int32_t* indices, float* out) {
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  size_t sort1 = 0, sort2 = 0, scan = 0;
  ANNC_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sort1, (const int64_t*)nullptr,
                                                  (int64_t*)nullptr, (const int32_t*)nullptr,
                                                  (int32_t*)nullptr, (int)n, 0, 64, s));
  ANNC_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sort2, (const int32_t*)nullptr,
                                                  (int32_t*)nullptr, (const int32_t*)nullptr,
                                                  (int32_t*)nullptr, (int)n, 0, 32, s));
  ANNC_HIP_TRY(hipcub::DeviceScan::InclusiveSum(nullptr, scan, (const int32_t*)nullptr,
                                                (int32_t*)nullptr, (int)n, s));
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t n8 = align(sizeof(int64_t) * (size_t)n), n4 = align(sizeof(int32_t) * (size_t)n);
  const size_t temp = align(std::max(sort1, std::max(sort2, scan)));
  char* ws = static_cast<char*>(stream_workspace(s, 3 * n8 + 9 * n4 + temp));
  if (!ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  int64_t* k_in = reinterpret_cast<int64_t*>(ws);
  int64_t* k_out = reinterpret_cast<int64_t*>(ws + n8);
  int64_t* run_key = reinterpret_cast<int64_t*>(ws + 2 * n8);
  char* w4 = ws + 3 * n8;
  int32_t* p_in = reinterpret_cast<int32_t*>(w4);
  int32_t* p_out = reinterpret_cast<int32_t*>(w4 + n4);
  int32_t* head = reinterpret_cast<int32_t*>(w4 + 2 * n4);
  int32_t* runid = reinterpret_cast<int32_t*>(w4 + 3 * n4);
  int32_t* first_pos = reinterpret_cast<int32_t*>(w4 + 4 * n4);
  int32_t* run_idx = reinterpret_cast<int32_t*>(w4 + 5 * n4);
  int32_t* first_sorted = reinterpret_cast<int32_t*>(w4 + 6 * n4);
  int32_t* order = reinterpret_cast<int32_t*>(w4 + 7 * n4);
  int32_t* rank_of_run = reinterpret_cast<int32_t*>(w4 + 8 * n4);
  void* tmp = w4 + 9 * n4;
  const dim3 grid((unsigned)ceil_div(n, kThreads));
  hipLaunchKernelGGL(extract_keys_kernel, grid, dim3(kThreads), 0, s, keys, stride, n, k_in, p_in);
  ANNC_HIP_TRY(hipGetLastError());
  ANNC_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(tmp, sort1, k_in, k_out, p_in, p_out, (int)n, 0,
                                                  64, s));
  hipLaunchKernelGGL(run_heads_kernel, grid, dim3(kThreads), 0, s, k_out, n, head, first_pos);
  ANNC_HIP_TRY(hipGetLastError());
  ANNC_HIP_TRY(hipcub::DeviceScan::InclusiveSum(tmp, scan, head, runid, (int)n, s));
  hipLaunchKernelGGL(run_first_kernel, grid, dim3(kThreads), 0, s, k_out, p_out, head, runid, n,
                     first_pos, run_idx, run_key);
  ANNC_HIP_TRY(hipGetLastError());
  ANNC_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(tmp, sort2, first_pos, first_sorted, run_idx,
                                                  order, (int)n, 0, 32, s));
  hipLaunchKernelGGL(rank_kernel, grid, dim3(kThreads), 0, s, order, run_key, runid, n,
                     rank_of_run, unique, num_unique);
  ANNC_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(indices_kernel, grid, dim3(kThreads), 0, s, p_out, runid, rank_of_run, n,
                     indices);
  ANNC_HIP_TRY(hipGetLastError());
  if (dim > 0) {
    hipLaunchKernelGGL(gather_unique_kernel, dim3((unsigned)ceil_div(n * dim, kThreads)),
                       dim3(kThreads), 0, s, table, rows, dim, unique, runid, n, out, status);
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
