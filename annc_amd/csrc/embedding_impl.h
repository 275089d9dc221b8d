// embedding_impl.h -- internal launchers shared by the embedding, hashing
// and TF-op entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace annc {

struct BagArgs {
  const float* table;
  int64_t rows;
  int64_t dim;
  const void* ids;
  int ids_is_64;
  const int64_t* offsets;
  const int32_t* perm;  // optional: row id of position j is ids[perm[j]]
  int64_t num_bags;
  int combiner;
  float* out;
  int64_t ldo;
  int* status;
};

// CSR bag reduction (sum or mean) in index order.
int launch_bag(const BagArgs& a, hipStream_t s);

// Min, max and sortedness of seg[i*stride], i < n (synchronises `s`).
int segment_scan(hipStream_t s, const int64_t* seg, int64_t stride, int64_t n, int64_t* min_out,
                 int64_t* max_out, bool* sorted);

// out[batch, dim] = segment reduction of data rows; positions whose segment
// id lies outside [0, batch) are skipped.  sorted_hint = 1 when the ids are
// known to be non-decreasing.  Workspace from the stream, status word of
// the stream.
int segment_reduce(hipStream_t s, const float* data, int64_t rows, int64_t dim,
                   const void* indices, int indices_is_64, const int64_t* seg, int64_t stride,
                   int64_t n, int combiner, int64_t batch, float* out, int sorted_hint);

// The path a segment reduction takes and the device workspace it needs.
struct SegPlan {
  enum Path { kSorted, kTwoLevel, kCounting, kRadix } path = kSorted;
  size_t bytes = 0;       // workspace bytes
  size_t temp_bytes = 0;  // radix sort temporary storage (kRadix)
  int end_bit = 0;        // radix sort key bits (kRadix)
};
int segment_reduce_plan(int64_t n, int64_t batch, int sorted_hint, hipStream_t s, SegPlan* plan);
// Runs `plan` with caller-provided workspace (plan.bytes, 256-byte aligned)
// and status word (bit 0 is set for a row id outside the data).  Allocates
// nothing.
int segment_reduce_run(hipStream_t s, const float* data, int64_t rows, int64_t dim,
                       const void* indices, int indices_is_64, const int64_t* seg, int64_t stride,
                       int64_t n, int combiner, int64_t batch, float* out, const SegPlan& plan,
                       void* workspace, int* status);

// Keys in first-occurrence order over a known small range (every key in
// [kmin, kmin + range)): unique[r] = the r-th distinct key by first position,
// indices[i] = the number of position i's key, *num_unique (device) = U.
// A table of `range` ints replaces the hash of annc_hip_unique_gather.
int first_occurrence_range(hipStream_t s, const int64_t* keys, int64_t stride, int64_t n,
                           int64_t kmin, int64_t range, int64_t* num_unique, int64_t* unique,
                           int32_t* indices);

// dst[i] = src[i] for i < n (int32 -> int64).
int widen_i32(hipStream_t s, const int32_t* src, int64_t n, int64_t* dst);

// KPFusedSparseSegmentReduceNonzero's output form of a dense [rows, dim]
// reduction (row r holds segment seg_of_row[r]): flags[i] = dense[i] != 0,
// incl = their inclusive scan (incl[count - 1] = the number of nonzeros),
// and with out_idx the nonzero coordinates ((segment) for one_d, else
// (segment, dim)) and values in row-major order, the first `cap` of them
// (out_idx and out_val hold cap entries).  tmp holds
// nonzero_scan_temp_bytes(count) bytes.
size_t nonzero_scan_temp_bytes(int64_t count);
int nonzero_compact(hipStream_t s, const float* dense, int64_t count, int64_t dim,
                    const int64_t* seg_of_row, int one_d, int32_t* flags, int32_t* incl, void* tmp,
                    size_t tmp_bytes, int64_t cap, int32_t* out_idx, float* out_val);
// The write step of nonzero_compact alone, over flags and incl it computed.
int nonzero_write(hipStream_t s, const float* dense, int64_t count, int64_t dim,
                  const int64_t* seg_of_row, int one_d, const int32_t* flags, const int32_t* incl,
                  int64_t cap, int32_t* out_idx, float* out_val);

int launch_sparse_embedding2(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                             const void* ids, int ids_is_64, int64_t n, int64_t fallback,
                             float* out);

int launch_pooling(hipStream_t s, const int64_t* ids, const float* gathered, int64_t m, int64_t k,
                   int64_t n, const int64_t* ss, const int64_t* sl, float* out);
// out[i] = sum(|x[i*m .. i*m+m)|) / m for i < n (the __reduce_mean target).
int launch_abs_mean(hipStream_t s, const float* x, int64_t m, int64_t n, float* out);

// Hash-bucket helpers (hash.hip).
struct StringsArgs {
  const char* bytes;
  const int64_t* offsets;
  int64_t n;
};
// Unsigned 64-bit division by an invariant divisor (round-up method of
// Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, fig. 4.1).
struct U64Divisor {
  uint64_t d;
  uint64_t magic;
  int shift;  // l - 1; d == 1 uses shift = -1
};
U64Divisor make_divisor(uint64_t d);

}  // namespace annc
