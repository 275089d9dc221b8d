// tf_ops.cpp -- C entry points mirroring ANNC's TensorFlow custom ops.
//
// TensorFlow is not part of this build, so each REGISTER_OP becomes one C
// function with the same inputs, attributes and OP_REQUIRES messages; the
// arithmetic runs on the GPU kernels of embedding.hip / hash.hip.  Operand
// pointers may be host or device memory; calls are synchronous.
#include <algorithm>
#include <cstring>
#include <map>
#include <vector>

#include "common.h"
#include "embedding_impl.h"

namespace annc {
int launch_bucket_strings(hipStream_t s, const char* bytes, const int64_t* offsets, int64_t n,
                          int64_t num_buckets, int nul, int64_t empty_value, int64_t* out);
int launch_gather_rows(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                       const int64_t* bucket, int64_t n, float* out);
int unique_gather(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                  const int64_t* keys, int64_t stride, int64_t n, int64_t* num_unique,
                  int64_t* unique, int32_t* indices, float* out);
int launch_broadcast3(hipStream_t s, const float* src, int64_t s0, int64_t s1, int64_t s2,
                      int64_t nz, int64_t m, int64_t n, float* dst);
int run_sparse_embedding(hipStream_t s, const int64_t* offsets, const int64_t* bucket, int64_t n,
                         int32_t* keep, int32_t* pos, int64_t* indices, int64_t* values,
                         uint8_t* empty, int64_t* num_values);

namespace {

int read_i32(const int32_t* src, int64_t count, int32_t* dst) {
  if (count <= 0) return ANNC_OK;
  if (is_device_ptr(src)) {
    ANNC_HIP_TRY(hipMemcpy(dst, src, sizeof(int32_t) * count, hipMemcpyDeviceToHost));
  } else {
    std::memcpy(dst, src, sizeof(int32_t) * count);
  }
  return ANNC_OK;
}

int write_i32(int32_t* dst, int32_t v) {
  if (!dst) return ANNC_OK;
  if (is_device_ptr(dst)) {
    ANNC_HIP_TRY(hipMemcpy(dst, &v, sizeof(v), hipMemcpyHostToDevice));
  } else {
    *dst = v;
  }
  return ANNC_OK;
}

// Total byte count of a strings operand = offsets[n].
int strings_bytes(const int64_t* offsets, int64_t n, int64_t* total) {
  return read_i64(offsets + n, 1, total);
}

// Hash-bucket embedding shared by the three dense-output ops.
int embed_hash_bucket(const char* bytes, const int64_t* offsets, int64_t batch,
                      const float* weight, int64_t rows, int64_t dim, int64_t num_buckets, int nul,
                      float* output) {
  ANNC_REQUIRE(num_buckets >= 1, "num_buckets must be >= 1");
  ANNC_REQUIRE(batch >= 0 && rows >= 0 && dim >= 0, "bad dimensions");
  if (batch == 0 || dim == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(bytes && offsets && weight && output, "null pointer");
  int64_t total = 0;
  int rc = strings_bytes(offsets, batch, &total);
  if (rc != ANNC_OK) return rc;
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const char* d_bytes = static_cast<const char*>(st.in(bytes, (size_t)(total > 0 ? total : 1)));
  const int64_t* d_off = static_cast<const int64_t*>(st.in(offsets, sizeof(int64_t) * (batch + 1)));
  const float* d_w = static_cast<const float*>(st.in(weight, sizeof(float) * rows * dim));
  float* d_out = static_cast<float*>(st.out(output, sizeof(float) * batch * dim));
  int64_t* bucket = static_cast<int64_t*>(st.scratch(sizeof(int64_t) * batch));
  if (st.status() != ANNC_OK) return st.status();
  rc = launch_bucket_strings(s, d_bytes, d_off, batch, num_buckets, nul, -1, bucket);
  if (rc == ANNC_OK) rc = launch_gather_rows(s, d_w, rows, dim, bucket, batch, d_out);
  if (rc != ANNC_OK) return rc;
  rc = st.finish();
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

}  // namespace
}  // namespace annc

namespace annc {
namespace {

// Device scratch of KPFusedSparseSegmentReduceNonzero, per thread and
// device.  Buffers grow as needed and, like the thread's pinned and staging
// buffers, are kept until the process ends (releasing them at thread exit
// could run after the HIP runtime has shut down).
struct DeviceBuf {
  char* p = nullptr;
  size_t size = 0;
  char* get(size_t bytes) {
    if (bytes <= size) return p;
    if (p) (void)hipFree(p);  // waits for the device: no earlier use is pending
    p = nullptr;
    size = 0;
    if (hipMalloc(&p, bytes) != hipSuccess) {
      p = nullptr;
      return nullptr;
    }
    size = bytes;
    return p;
  }
};

struct NzScratch {
  DeviceBuf uniq_buf, dense_buf;  // segments by first appearance; dense, flags, incl, scan temp
};
thread_local std::map<int, NzScratch> t_nz;

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace
}  // namespace annc

extern "C" {

int annc_kp_fused_sparse_segment_reduce(const float* data, int data_rank, const int64_t* data_dims,
                                        const void* indices, int indices_is_64,
                                        int64_t num_indices, const int64_t* slice_input,
                                        int slice_rank, const int64_t* slice_dims,
                                        const int32_t* begin, int64_t begin_elems,
                                        const int32_t* begin_1, int64_t begin_1_elems,
                                        int combiner, int64_t* out_rows, float* output,
                                        int32_t* slice_output) {
  using namespace annc;
  // OpKernel constructor (embedding_fused_sparse_segment_reduce.cc:33-34).
  ANNC_REQUIRE(combiner == 0 || combiner == 1, "combiner must be 0 or 1");
  // Compute() checks, same order and text (:45-57).
  ANNC_REQUIRE(data_rank == 2, "input must be 2-D");
  ANNC_REQUIRE(slice_rank == 2, "slice input must be 2-D");
  ANNC_REQUIRE(begin_elems == 2, "begin must have 2 elements");
  ANNC_REQUIRE(begin_1_elems == 1, "begin_1 must have 1 element");
  ANNC_REQUIRE(data_dims && slice_dims && begin && begin_1, "null shape operand");
  int32_t b[2], b1 = 0;
  int rc = read_i32(begin, 2, b);
  if (rc == ANNC_OK) rc = read_i32(begin_1, 1, &b1);
  if (rc != ANNC_OK) return rc;
  const int64_t rows = data_dims[0], dim = data_dims[1];
  const int32_t col = b[1];
  ANNC_REQUIRE(col >= 0 && col < slice_dims[1], "Column index out of range");
  ANNC_REQUIRE(num_indices == slice_dims[0],
               "indices and slice_input.dim_zie(0) should have same size");
  ANNC_REQUIRE(num_indices == 0 || (indices && slice_input), "null operand");

  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const int64_t* d_slice = static_cast<const int64_t*>(
      st.in(slice_input, sizeof(int64_t) * (size_t)(slice_dims[0] * slice_dims[1])));
  if (st.status() != ANNC_OK) return st.status();
  int64_t seg_min = 0, seg_max = 0;
  bool sorted = true;
  rc = segment_scan(s, d_slice + col, slice_dims[1], num_indices, &seg_min, &seg_max, &sorted);
  if (rc != ANNC_OK) return rc;
  // max_seg_id starts at 0 (:64-71): batch >= 1 even with no indices.
  const int64_t max_seg = num_indices > 0 && seg_max > 0 ? seg_max : 0;
  ANNC_REQUIRE(num_indices == 0 || seg_min >= 0, "segment id %lld out of range",
               (long long)seg_min);
  const int64_t batch = max_seg + 1;
  if (out_rows) *out_rows = batch;
  if (!output) return set_error(ANNC_OK, "");

  const float* d_data = static_cast<const float*>(st.in(data, sizeof(float) * rows * dim));
  const void* d_idx = st.in(indices, (indices_is_64 ? 8 : 4) * (size_t)num_indices);
  float* d_out = static_cast<float*>(st.out(output, sizeof(float) * batch * dim));
  if (st.status() != ANNC_OK) return st.status();
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  ANNC_HIP_TRY(hipMemsetAsync(status, 0, sizeof(int), s));
  if (dim > 0) {
    rc = segment_reduce(s, d_data, rows, dim, d_idx, indices_is_64, d_slice + col, slice_dims[1],
                        num_indices, combiner, batch, d_out, sorted ? 1 : 0);
    if (rc != ANNC_OK) return rc;
  }
  rc = st.finish();
  if (rc != ANNC_OK) return rc;
  int bad = 0;
  rc = read_back(s, {{&bad, status, sizeof(int)}});
  if (rc != ANNC_OK) return rc;
  if (bad) {
    ANNC_HIP_TRY(hipMemset(status, 0, sizeof(int)));
    return set_error(ANNC_INVALID_ARGUMENT, "indices out of range of the %lld data rows",
                     (long long)rows);
  }
  // slice_output: batch when begin_1 == 0, else the embedding size (:81-83).
  rc = write_i32(slice_output, b1 == 0 ? static_cast<int32_t>(batch) : static_cast<int32_t>(dim));
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}


int annc_kp_fused_sparse_segment_reduce_nonzero(
    const float* data, int data_rank, const int64_t* data_dims, const void* indices,
    int indices_is_64, int64_t num_indices, const int64_t* slice_input, int slice_rank,
    const int64_t* slice_dims, const int32_t* begin, int64_t begin_elems, int combiner,
    int32_t* output_shape, int64_t* num_nonzero, int32_t* output_indices,
    float* output_nonzero) {
  using namespace annc;
  // OpKernel constructor and Compute() checks, same order and text
  // (embedding_fused_sparse_segment_reduce_nonzero.cc:33-57).
  ANNC_REQUIRE(combiner == 0 || combiner == 1, "combiner must be 0 or 1");
  ANNC_REQUIRE(data_rank == 1 || data_rank == 2, "Input data must be a 1-D vector or 2-D matrix");
  ANNC_REQUIRE(slice_rank == 2, "slice input must be 2-D");
  ANNC_REQUIRE(begin_elems == 2, "begin must have 2 elements");
  ANNC_REQUIRE(data_dims && slice_dims && begin && num_nonzero, "null shape operand");
  int32_t b[2];
  int rc = read_i32(begin, 2, b);
  if (rc != ANNC_OK) return rc;
  const int32_t col = b[1];
  ANNC_REQUIRE(col >= 0 && col < slice_dims[1], "Column index out of range");
  ANNC_REQUIRE(num_indices == slice_dims[0],
               "indices and slice_input.dim_size(0) should have same size");
  ANNC_REQUIRE(num_indices == 0 || (indices && slice_input), "null operand");
  ANNC_REQUIRE(num_indices < INT32_MAX, "too many indices");
  const int64_t rows = data_dims[0], dim = data_rank == 2 ? data_dims[1] : 1;
  const int one_d = data_rank == 1 ? 1 : 0;
  // phase 2 (outputs given) takes the phase-1 count as the output size
  const bool write = output_indices != nullptr;
  ANNC_REQUIRE(!write || output_nonzero != nullptr || *num_nonzero == 0, "null output");
  const int64_t cap = write ? *num_nonzero : 0;

  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  int device = 0;
  ANNC_HIP_TRY(hipGetDevice(&device));
  NzScratch& nz = t_nz[device];
  // Phase 2 recomputes from the operands (they may have changed since phase
  // 1); the result is deterministic, so an unchanged input gives phase 1's
  // count.
  Staging st(s);
  const int64_t stride = slice_dims[1];
  const int64_t* d_slice = static_cast<const int64_t*>(
      st.in(slice_input, sizeof(int64_t) * (size_t)(slice_dims[0] * stride)));
  if (st.status() != ANNC_OK) return st.status();
  int64_t seg_min = 0, seg_max = 0;
  bool sorted = true;
  rc = segment_scan(s, d_slice + col, stride, num_indices, &seg_min, &seg_max, &sorted);
  if (rc != ANNC_OK) return rc;
  // max_seg_id starts at 0 (:63-71)
  const int64_t batch = (num_indices > 0 && seg_max > 0 ? seg_max : 0) + 1;
  if (output_shape) {
    rc = write_i32(output_shape, static_cast<int32_t>(batch));
    if (rc == ANNC_OK && !one_d) rc = write_i32(output_shape + 1, static_cast<int32_t>(dim));
    if (rc != ANNC_OK) return rc;
  }
  if (num_indices == 0 || dim == 0) {
    *num_nonzero = 0;
    return set_error(ANNC_OK, "");
  }

  // segments in order of first appearance, and each position's rank among them
  int64_t* d_nu = static_cast<int64_t*>(st.scratch(sizeof(int64_t)));
  int64_t* d_uniq = reinterpret_cast<int64_t*>(nz.uniq_buf.get(sizeof(int64_t) * num_indices));
  int32_t* d_slot = static_cast<int32_t*>(st.scratch(sizeof(int32_t) * num_indices));
  int64_t* d_slot64 = static_cast<int64_t*>(st.scratch(sizeof(int64_t) * num_indices));
  if (!d_nu || !d_uniq || !d_slot || !d_slot64)
    return set_error(ANNC_RESOURCE_EXHAUSTED, "scratch allocation failed");
  // segment ids spanning a small range (the scan gave min and max) index a
  // table directly; others go through the hash table of KPFusedGather
  const uint64_t range = static_cast<uint64_t>(seg_max) - static_cast<uint64_t>(seg_min) + 1;
  if (range <= static_cast<uint64_t>(std::max<int64_t>(4 * num_indices, int64_t(1) << 16)) &&
      range <= (uint64_t(1) << 26))
    rc = first_occurrence_range(s, d_slice + col, stride, num_indices, seg_min,
                                static_cast<int64_t>(range), d_nu, d_uniq, d_slot);
  else
    rc = annc_hip_unique_gather(s, nullptr, 0, 0, d_slice + col, stride, num_indices, d_nu,
                                d_uniq, d_slot, nullptr);
  if (rc != ANNC_OK) return rc;
  int64_t nseg = 0;
  rc = read_back(s, {{&nseg, d_nu, sizeof(int64_t)}});
  if (rc != ANNC_OK) return rc;
  rc = widen_i32(s, d_slot, num_indices, d_slot64);
  if (rc != ANNC_OK) return rc;

  // per-segment reduction in index order, rows in first-appearance order
  const float* d_data = static_cast<const float*>(st.in(data, sizeof(float) * rows * dim));
  const void* d_idx = st.in(indices, (indices_is_64 ? 8 : 4) * (size_t)num_indices);
  const int64_t count = nseg * dim;
  // dense values, flags, their scan and the scan's temporary storage
  const size_t vb = align256(sizeof(float) * (size_t)count);
  const size_t tmp_bytes = nonzero_scan_temp_bytes(count);
  char* db = nz.dense_buf.get(3 * vb + align256(std::max<size_t>(tmp_bytes, 1)));
  float* d_dense = reinterpret_cast<float*>(db);
  int32_t* d_flags = db ? reinterpret_cast<int32_t*>(db + vb) : nullptr;
  int32_t* d_incl = db ? reinterpret_cast<int32_t*>(db + 2 * vb) : nullptr;
  void* d_tmp = db ? db + 3 * vb : nullptr;
  if (st.status() != ANNC_OK) return st.status();
  if (!d_dense || !d_flags || !d_incl || !d_tmp)
    return set_error(ANNC_RESOURCE_EXHAUSTED, "scratch allocation failed");
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  ANNC_HIP_TRY(hipMemsetAsync(status, 0, sizeof(int), s));
  rc = segment_reduce(s, d_data, rows, dim, d_idx, indices_is_64, d_slot64, 1, num_indices, combiner,
                      nseg, d_dense, 0);
  if (rc != ANNC_OK) return rc;

  int32_t* d_out_idx = nullptr;
  float* d_out_val = nullptr;
  if (write && cap > 0) {
    d_out_idx = static_cast<int32_t*>(st.out(output_indices, sizeof(int32_t) * cap * (one_d ? 1 : 2)));
    d_out_val = static_cast<float*>(st.out(output_nonzero, sizeof(float) * cap));
    if (st.status() != ANNC_OK) return st.status();
  }
  rc = nonzero_compact(s, d_dense, count, dim, d_uniq, one_d, d_flags, d_incl, d_tmp, tmp_bytes,
                       cap, d_out_idx, d_out_val);
  if (rc != ANNC_OK) return rc;
  int32_t nnz = 0;
  int bad = 0;
  rc = read_back(s, {{&nnz, d_incl + (count - 1), sizeof(int32_t)}, {&bad, status, sizeof(int)}});
  if (rc != ANNC_OK) return rc;
  if (bad) {
    ANNC_HIP_TRY(hipMemset(status, 0, sizeof(int)));
    return set_error(ANNC_INVALID_ARGUMENT, "indices out of range of the %lld data rows",
                     (long long)rows);
  }
  // a phase-2 buffer must be what phase 1 counted (the result is deterministic)
  ANNC_REQUIRE(!write || nnz == cap, "output size %lld differs from the %lld nonzero values",
               (long long)cap, (long long)nnz);
  if (write && cap > 0) {
    rc = st.finish();
    if (rc != ANNC_OK) return rc;
  }
  *num_nonzero = nnz;
  return set_error(ANNC_OK, "");
}

int annc_kp_fused_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets,
                                             int64_t batch, const float* weight, int64_t rows,
                                             int64_t dim, int64_t num_buckets, int combiner,
                                             float* output) {
  (void)combiner;  // accepted and ignored (fused_embedding_with_hash_bucket.cc:61-77)
  using namespace annc;
  ANNC_REQUIRE(num_buckets <= rows || batch == 0,
               "num_buckets (%lld) exceeds the weight rows (%lld)", (long long)num_buckets,
               (long long)rows);
  return embed_hash_bucket(bytes, offsets, batch, weight, rows, dim, num_buckets, 0, output);
}

int annc_kp_fused_dnn_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets,
                                                 int64_t batch, const float* weight, int64_t rows,
                                                 int64_t dim, int64_t num_buckets,
                                                 float* output) {
  return annc::embed_hash_bucket(bytes, offsets, batch, weight, rows, dim, num_buckets, 1, output);
}

int annc_kp_fused_linear_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets,
                                                    int64_t batch, const float* weight,
                                                    int64_t rows, int64_t dim,
                                                    int64_t num_buckets, float* output) {
  return annc::embed_hash_bucket(bytes, offsets, batch, weight, rows, dim, num_buckets, 1, output);
}

int annc_kp_fused_sparse_embedding(const char* bytes, const int64_t* offsets, int64_t n,
                                   int64_t num_buckets, int64_t* output_indices,
                                   int64_t* output_values, uint8_t* empty_row_indicator,
                                   int64_t* output_shape, int64_t* num_values) {
  using namespace annc;
  ANNC_REQUIRE(num_buckets >= 1, "num_buckets must be >= 1");
  ANNC_REQUIRE(n >= 0, "negative count");
  ANNC_REQUIRE(num_values != nullptr, "null num_values");
  int64_t shape[2] = {n, 1};
  if (output_shape) {
    if (is_device_ptr(output_shape)) {
      ANNC_HIP_TRY(hipMemcpy(output_shape, shape, sizeof(shape), hipMemcpyHostToDevice));
    } else {
      output_shape[0] = n;
      output_shape[1] = 1;
    }
  }
  if (n == 0) {
    *num_values = 0;
    return set_error(ANNC_OK, "");
  }
  ANNC_REQUIRE(bytes && offsets && output_indices && output_values && empty_row_indicator,
               "null pointer");
  int64_t total = 0;
  int rc = strings_bytes(offsets, n, &total);
  if (rc != ANNC_OK) return rc;
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const char* d_bytes = static_cast<const char*>(st.in(bytes, (size_t)(total > 0 ? total : 1)));
  const int64_t* d_off = static_cast<const int64_t*>(st.in(offsets, sizeof(int64_t) * (n + 1)));
  int64_t* d_idx = static_cast<int64_t*>(st.out(output_indices, sizeof(int64_t) * 2 * n));
  int64_t* d_val = static_cast<int64_t*>(st.out(output_values, sizeof(int64_t) * n));
  uint8_t* d_empty = static_cast<uint8_t*>(st.out(empty_row_indicator, (size_t)n));
  int64_t* bucket = static_cast<int64_t*>(st.scratch(sizeof(int64_t) * n));
  int32_t* keep = static_cast<int32_t*>(st.scratch(sizeof(int32_t) * n));
  int32_t* pos = static_cast<int32_t*>(st.scratch(sizeof(int32_t) * n));
  if (st.status() != ANNC_OK) return st.status();
  rc = launch_bucket_strings(s, d_bytes, d_off, n, num_buckets, 1, 0, bucket);
  if (rc == ANNC_OK)
    rc = run_sparse_embedding(s, d_off, bucket, n, keep, pos, d_idx, d_val, d_empty, num_values);
  if (rc != ANNC_OK) return rc;
  rc = st.finish();
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

int annc_kp_fused_gather(const float* data, int data_rank, const int64_t* data_dims,
                         const int64_t* slice_input, int slice_rank, const int64_t* slice_dims,
                         const int32_t* begin, int64_t begin_elems, int64_t* num_unique,
                         int64_t* out_unique, int32_t* out_indices, float* out_data) {
  using namespace annc;
  // Compute() checks, same order and text (embedding_fused_gather.cc:34-42);
  // the reference reports them as errors::Internal.
  if (slice_rank != 2) return set_error(ANNC_INTERNAL, "Input key must be 2D");
  if (data_rank != 2) return set_error(ANNC_INTERNAL, "Embedding table shape must be 2D");
  if (begin_elems != 2) return set_error(ANNC_INTERNAL, "begin must be same as keys rank");
  ANNC_REQUIRE(data_dims && slice_dims && begin && num_unique, "null operand");
  int32_t b[2];
  int rc = read_i32(begin, 2, b);
  if (rc != ANNC_OK) return rc;
  const int32_t col = b[1];
  if (col < 0 || col >= slice_dims[1])
    return set_error(ANNC_INTERNAL, "slice cols out of keys range");
  const int64_t rows = data_dims[0], dim = data_dims[1], n = slice_dims[0];
  ANNC_REQUIRE(rows >= 0 && dim >= 0 && n >= 0, "bad dimensions");
  ANNC_REQUIRE(n < (int64_t(1) << 31) - 1, "too many keys");
  if (n == 0) {
    *num_unique = 0;
    return set_error(ANNC_OK, "");
  }
  ANNC_REQUIRE(slice_input && (data || rows * dim == 0), "null operand");
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  ANNC_HIP_TRY(hipMemsetAsync(status, 0, sizeof(int), s));  // start from a clear status word
  Staging st(s);
  const float* d_data =
      static_cast<const float*>(st.in(data, sizeof(float) * (size_t)(rows * dim > 0 ? rows * dim : 1)));
  const int64_t* d_keys =
      static_cast<const int64_t*>(st.in(slice_input, sizeof(int64_t) * (size_t)(n * slice_dims[1])));
  int64_t* d_nu = static_cast<int64_t*>(st.scratch(sizeof(int64_t)));
  int64_t* d_uniq = static_cast<int64_t*>(st.scratch(sizeof(int64_t) * (size_t)n));
  int32_t* d_idx = static_cast<int32_t*>(st.scratch(sizeof(int32_t) * (size_t)n));
  float* d_out = static_cast<float*>(st.scratch(sizeof(float) * (size_t)(n * (dim > 0 ? dim : 1))));
  if (st.status() != ANNC_OK) return st.status();
  rc = unique_gather(s, d_data, rows, dim, d_keys + col, slice_dims[1], n, d_nu, d_uniq, d_idx,
                     d_out);
  if (rc != ANNC_OK) return rc;
  // the status word and the unique count in one synchronisation
  int bad = 0;
  int64_t u = 0;
  rc = read_back(s, {{&bad, status, sizeof(int)}, {&u, d_nu, sizeof(u)}});
  if (rc != ANNC_OK) return rc;
  if (bad) {
    ANNC_HIP_TRY(hipMemset(status, 0, sizeof(int)));
    return set_error(ANNC_INTERNAL, "idx out of table range");
  }
  *num_unique = u;
  // the outputs are sized by u: copied once it is known, then one wait
  if (out_unique)
    ANNC_HIP_TRY(hipMemcpyAsync(out_unique, d_uniq, sizeof(int64_t) * (size_t)u, hipMemcpyDefault, s));
  if (out_indices)
    ANNC_HIP_TRY(hipMemcpyAsync(out_indices, d_idx, sizeof(int32_t) * (size_t)n, hipMemcpyDefault, s));
  if (out_data && u * dim > 0)
    ANNC_HIP_TRY(hipMemcpyAsync(out_data, d_out, sizeof(float) * (size_t)(u * dim), hipMemcpyDefault, s));
  ANNC_HIP_TRY(hipStreamSynchronize(s));
  return set_error(ANNC_OK, "");
}

int annc_kp_fused_batch_matmul_add_sigmoid(const float* lhs, int lhs_rank,
                                           const int64_t* lhs_dims, const float* rhs, int rhs_rank,
                                           const int64_t* rhs_dims, const float* bias,
                                           int bias_rank, const int64_t* bias_dims,
                                           float* output) {
  using namespace annc;
  // Compute() checks, same order and text (fused_batchmatmul_add_sigmoid.cc:
  // Compute and BuildBiasInfo).
  ANNC_REQUIRE(lhs_rank == 3, "lhs must be rank 3");
  ANNC_REQUIRE(rhs_rank == 2 || rhs_rank == 3, "rhs must be rank 2 or 3");
  ANNC_REQUIRE(bias_rank >= 0 && bias_rank <= 3, "bias rank must be <= 3");
  ANNC_REQUIRE(lhs_dims && rhs_dims && (bias_rank == 0 || bias_dims), "null shape operand");
  const int64_t batch = lhs_dims[0], m = lhs_dims[1], k = lhs_dims[2];
  const bool rhs_batched = rhs_rank == 3;
  ANNC_REQUIRE(!rhs_batched || rhs_dims[0] == batch, "lhs/rhs batch mismatch");
  ANNC_REQUIRE(rhs_dims[rhs_batched ? 1 : 0] == k, "lhs/rhs contracting dim mismatch");
  const int64_t n = rhs_dims[rhs_batched ? 2 : 1];
  int64_t bd[3] = {1, 1, 1};
  for (int i = 0; i < bias_rank; ++i) bd[3 - bias_rank + i] = bias_dims[i];
  ANNC_REQUIRE((bd[0] == 1 || bd[0] == batch) && (bd[1] == 1 || bd[1] == m) &&
                   (bd[2] == 1 || bd[2] == n),
               "bias shape is not broadcast-compatible");
  if (batch == 0 || m == 0 || n == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(lhs && rhs && bias && output, "null operand");
  const int64_t s2 = bd[2] == 1 ? 0 : 1;
  const int64_t s1 = bd[1] == 1 ? 0 : bd[2];
  const int64_t s0 = bd[0] == 1 ? 0 : bd[1] * bd[2];
  const int64_t nz = bd[0];  // 1 or batch: the materialised addend's batch
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const size_t f = sizeof(float);
  const float* d_lhs = static_cast<const float*>(st.in(lhs, f * (size_t)(batch * m * k)));
  const float* d_rhs = static_cast<const float*>(
      st.in(rhs, f * (size_t)((rhs_batched ? batch : 1) * k * n)));
  const float* d_bias = static_cast<const float*>(st.in(bias, f * (size_t)(bd[0] * bd[1] * bd[2])));
  float* d_out = static_cast<float*>(st.out(output, f * (size_t)(batch * m * n)));
  float* addend = static_cast<float*>(st.scratch(f * (size_t)(nz * m * n)));
  if (st.status() != ANNC_OK) return st.status();
  int rc = launch_broadcast3(s, d_bias, s0, s1, s2, nz, m, n, addend);
  if (rc == ANNC_OK)
    rc = annc_hip_gemm(s, batch, m, n, k, d_lhs, k, m * k, d_rhs, n, rhs_batched ? k * n : 0, 0,
                       addend, n, nz > 1 ? m * n : 0, nullptr, ANNC_EPI_SIGMOID, d_out, n, m * n);
  if (rc != ANNC_OK) return rc;
  rc = st.finish();
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

}  // extern "C"
