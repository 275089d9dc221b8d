/*
 * annc_oracle.c -- CPU restatement of ANNC's fused-operator hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU library is
 * compared against; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Nothing in the product (annc_amd/) links or
 * calls it.
 *
 * Every function follows a reference file:line (paths relative to the ANNC
 * source tree).  How each one is pinned:
 *   ora_fingerprint64      published known-answer vectors (TensorFlow,
 *                          Guava, BigQuery, pyfarmhash) for lengths 0-16,
 *                          17-32 and >64; the 33-64 byte branch has no
 *                          published vector available offline: parity
 *                          unpinned for that branch.
 *   ora_segment_reduce     reference gtest golden vectors
 *                          (embedding_fused_sparse_segment_reduce_test.cc:57-101,
 *                          and the nonzero op's goldens,
 *                          embedding_fused_sparse_segment_reduce_nonzero_test.cc:56-239)
 *                          and brute force in tests/.
 *   ora_segment_reduce_nonzero
 *                          reference gtest golden vectors
 *                          (embedding_fused_sparse_segment_reduce_nonzero_test.cc:56-239)
 *                          and, on random inputs, the listing of
 *                          ora_segment_reduce's dense result in tests/.
 *   ora_embedding_bag      same order as ora_segment_reduce (CSR form);
 *                          checked equal to it in tests/.
 *   ora_pooling            brute force on tiny inputs in tests/.
 *   ora_reduce_mean        numpy's sum of |x| per run (float64) in tests/.
 *   ora_hash_bucket_int64  decimal text checked against Python's str(int);
 *                          the hash as ora_fingerprint64.
 *   ora_embedding_with_hash_bucket, ora_dnn_embedding_with_hash_bucket,
 *   ora_sparse_embedding   closed forms over the pinned hash in tests/
 *                          (empty string, NUL-terminated prefix, bucket past
 *                          the rows, the bucket-0 quirk), with planted
 *                          mistakes the checks must catch.
 *   ora_hashed_embedding_bags
 *                          equal, in tests/, to the per-field composition of
 *                          ora_hash_bucket_int64 and ora_embedding_bag on
 *                          ragged multi-field inputs, with planted field
 *                          mix-ups the check must catch.
 *   ora_batch_matmul_add_sigmoid
 *                          float64 closed form (numpy matmul + broadcast) on
 *                          the reference test's shapes and inputs
 *                          (fused_batchmatmul_add_sigmoid_test.cc:140-204).
 *   ora_fused_gather       reference gtest golden vector
 *                          (embedding_fused_gather_test.cc:111-128) and
 *                          numpy.unique(return_index, return_inverse) in tests/.
 *   ora_sgemm & wrappers   OpenBLAS 0.3.29 sgemm (the reference's pinned
 *                          math library, third_party/repo.bzl:7) loaded
 *                          from numpy's bundled scipy_openblas64_; checked
 *                          against float64 closed forms in tests/.
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================== */
/* FarmHash Fingerprint64 = farmhashna::Hash64 (google/farmhash, the        */
/* @farmhash_archive TensorFlow 2.15 builds; used by                         */
/* python/tensorflow/kernels/fused_embedding_with_hash_bucket.cc:63 through */
/* util::Fingerprint64).  Restated from the published algorithm.            */
/* ======================================================================== */
static const uint64_t kK0 = 0xc3a5c85c97cb3127ULL;
static const uint64_t kK1 = 0xb492b66fbe98f273ULL;
static const uint64_t kK2 = 0x9ae16a3b2f90404fULL;

static uint64_t ld64(const char* p) { uint64_t r; memcpy(&r, p, 8); return r; }
static uint32_t ld32(const char* p) { uint32_t r; memcpy(&r, p, 4); return r; }
static uint64_t rotr(uint64_t v, int s) { return s == 0 ? v : ((v >> s) | (v << (64 - s))); }
static uint64_t shift_mix(uint64_t v) { return v ^ (v >> 47); }

static uint64_t hash_len16(uint64_t u, uint64_t v, uint64_t mul) {
  uint64_t a = (u ^ v) * mul;
  a ^= (a >> 47);
  uint64_t b = (v ^ a) * mul;
  b ^= (b >> 47);
  return b * mul;
}

static uint64_t hash_0_to_16(const char* s, size_t len) {
  if (len >= 8) {
    uint64_t mul = kK2 + len * 2;
    uint64_t a = ld64(s) + kK2;
    uint64_t b = ld64(s + len - 8);
    uint64_t c = rotr(b, 37) * mul + a;
    uint64_t d = (rotr(a, 25) + b) * mul;
    return hash_len16(c, d, mul);
  }
  if (len >= 4) {
    uint64_t mul = kK2 + len * 2;
    uint64_t a = ld32(s);
    return hash_len16(len + (a << 3), ld32(s + len - 4), mul);
  }
  if (len > 0) {
    uint8_t a = (uint8_t)s[0], b = (uint8_t)s[len >> 1], c = (uint8_t)s[len - 1];
    uint32_t y = (uint32_t)a + ((uint32_t)b << 8);
    uint32_t z = (uint32_t)len + ((uint32_t)c << 2);
    return shift_mix(y * kK2 ^ z * kK0) * kK2;
  }
  return kK2;
}

static uint64_t hash_17_to_32(const char* s, size_t len) {
  uint64_t mul = kK2 + len * 2;
  uint64_t a = ld64(s) * kK1;
  uint64_t b = ld64(s + 8);
  uint64_t c = ld64(s + len - 8) * mul;
  uint64_t d = ld64(s + len - 16) * kK2;
  return hash_len16(rotr(a + b, 43) + rotr(c, 30) + d, a + rotr(b + kK2, 18) + c, mul);
}

static uint64_t hash_33_to_64(const char* s, size_t len) {
  uint64_t mul = kK2 + len * 2;
  uint64_t a = ld64(s) * kK2;
  uint64_t b = ld64(s + 8);
  uint64_t c = ld64(s + len - 8) * mul;
  uint64_t d = ld64(s + len - 16) * kK2;
  uint64_t y = rotr(a + b, 43) + rotr(c, 30) + d;
  uint64_t z = hash_len16(y, a + rotr(b + kK2, 18) + c, mul);
  uint64_t e = ld64(s + 16) * mul;
  uint64_t f = ld64(s + 24);
  uint64_t g = (y + ld64(s + len - 32)) * mul;
  uint64_t h = (z + ld64(s + len - 24)) * mul;
  return hash_len16(rotr(e + f, 43) + rotr(g, 30) + h, e + rotr(f + a, 18) + g, mul);
}

typedef struct { uint64_t first, second; } u64pair;

static u64pair weak32(uint64_t w, uint64_t x, uint64_t y, uint64_t z, uint64_t a, uint64_t b) {
  a += w;
  b = rotr(b + a + z, 21);
  uint64_t c = a;
  a += x;
  a += y;
  b += rotr(a, 44);
  u64pair r = {a + z, b + c};
  return r;
}

static u64pair weak32_at(const char* s, uint64_t a, uint64_t b) {
  return weak32(ld64(s), ld64(s + 8), ld64(s + 16), ld64(s + 24), a, b);
}

uint64_t ora_fingerprint64(const char* s, size_t len) {
  const uint64_t seed = 81;
  if (len <= 16) return hash_0_to_16(s, len);
  if (len <= 32) return hash_17_to_32(s, len);
  if (len <= 64) return hash_33_to_64(s, len);
  uint64_t x = seed;
  uint64_t y = seed * kK1 + 113;
  uint64_t z = shift_mix(y * kK2 + 113) * kK2;
  u64pair v = {0, 0}, w = {0, 0};
  x = x * kK2 + ld64(s);
  const char* end = s + ((len - 1) / 64) * 64;
  const char* last64 = end + ((len - 1) & 63) - 63;
  do {
    x = rotr(x + y + v.first + ld64(s + 8), 37) * kK1;
    y = rotr(y + v.second + ld64(s + 48), 42) * kK1;
    x ^= w.second;
    y += v.first + ld64(s + 40);
    z = rotr(z + w.first, 33) * kK1;
    v = weak32_at(s, v.second * kK1, x + w.first);
    w = weak32_at(s + 32, z + w.second, y + ld64(s + 16));
    uint64_t t = z; z = x; x = t;
    s += 64;
  } while (s != end);
  uint64_t mul = kK1 + ((z & 0xff) << 1);
  s = last64;
  w.first += ((len - 1) & 63);
  v.first += w.first;
  w.first += v.first;
  x = rotr(x + y + v.first + ld64(s + 8), 37) * mul;
  y = rotr(y + v.second + ld64(s + 48), 42) * mul;
  x ^= w.second * 9;
  y += v.first * 9 + ld64(s + 40);
  z = rotr(z + w.first, 33) * mul;
  v = weak32_at(s, v.second * mul, x + w.first);
  w = weak32_at(s + 32, z + w.second, y + ld64(s + 16));
  { uint64_t t = z; z = x; x = t; }
  return hash_len16(hash_len16(v.first, w.first, mul) + shift_mix(y) * kK0 + z,
                    hash_len16(v.second, w.second, mul) + x, mul);
}

/* Length of the string for hashing: the whole [offsets[i], offsets[i+1])
 * span, or its NUL-terminated prefix (tensorflow::Fingerprint64(const char*)
 * as called at fused_dnn_embedding_with_hash_bucket.cc:30). */
static size_t str_len(const char* p, int64_t span, int nul_terminated) {
  if (!nul_terminated) return (size_t)span;
  size_t n = 0;
  while ((int64_t)n < span && p[n] != '\0') ++n;
  return n;
}

void ora_fingerprint64_batch(const char* bytes, const int64_t* offsets, int64_t n,
                             int nul_terminated, uint64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    const char* p = bytes + offsets[i];
    out[i] = ora_fingerprint64(p, str_len(p, offsets[i + 1] - offsets[i], nul_terminated));
  }
}

/* AsString(int64) with default attributes: "%lld". */
int ora_format_int64(int64_t v, char* buf) {
  return snprintf(buf, 24, "%lld", (long long)v);
}

/* StringToHashBucketFast: Fingerprint64(s) % num_buckets as uint64. */
void ora_hash_bucket_strings(const char* bytes, const int64_t* offsets, int64_t n,
                             int64_t num_buckets, int nul_terminated, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    const char* p = bytes + offsets[i];
    uint64_t h = ora_fingerprint64(p, str_len(p, offsets[i + 1] - offsets[i], nul_terminated));
    out[i] = (int64_t)(h % (uint64_t)num_buckets);
  }
}

void ora_hash_bucket_int64(const int64_t* ids, int64_t n, int64_t num_buckets, int64_t* out) {
  char buf[32];
  for (int64_t i = 0; i < n; ++i) {
    int len = ora_format_int64(ids[i], buf);
    out[i] = (int64_t)(ora_fingerprint64(buf, (size_t)len) % (uint64_t)num_buckets);
  }
}

/* ======================================================================== */
/* Segment reduction (KPFusedSparseSegmentReduceOp::Compute,                */
/* annc/tensorflow/kernels/embedding_fused_sparse_segment_reduce.cc:77-151): */
/* out zeroed; for i in index order out[seg_i, d] += data[idx_i, d]; mean:  */
/* out[seg, d] *= 1.0f / count.                                             */
/* ======================================================================== */
static int64_t idx_at(const void* p, int is64, int64_t i) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

void ora_segment_reduce(const float* data, int64_t rows, int64_t dim, const void* indices,
                        int idx64, const int64_t* seg, int64_t seg_stride, int64_t n,
                        int combiner, int64_t batch, float* out) {
  (void)rows;
  memset(out, 0, sizeof(float) * (size_t)(batch * dim));
  int32_t* counts = (int32_t*)calloc((size_t)(batch > 0 ? batch : 1), sizeof(int32_t));
  for (int64_t i = 0; i < n; ++i) {
    int64_t s = seg[i * seg_stride];
    int64_t r = idx_at(indices, idx64, i);
    counts[s] += 1;
    float* o = out + s * dim;
    const float* x = data + r * dim;
    for (int64_t d = 0; d < dim; ++d) o[d] += x[d];
  }
  if (combiner == 1) {
    for (int64_t s = 0; s < batch; ++s) {
      if (counts[s] > 0) {
        const float inv = 1.0f / (float)counts[s];
        float* o = out + s * dim;
        for (int64_t d = 0; d < dim; ++d) o[d] *= inv;
      }
    }
  }
  free(counts);
}

/* CSR form of the same reduction: bag b covers ids[offsets[b]..offsets[b+1]).
 * nthreads > 1 splits bags across OpenMP threads; each bag keeps its
 * sequential order, so the result does not depend on the thread count. */
void ora_embedding_bag(const float* table, int64_t rows, int64_t dim, const void* ids,
                       int idx64, const int64_t* offsets, int64_t nbags, int combiner,
                       float* out, int64_t ldo, int nthreads) {
  (void)rows;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#else
  (void)nthreads;
#endif
  for (int64_t b = 0; b < nbags; ++b) {
    float* o = out + b * ldo;
    for (int64_t d = 0; d < dim; ++d) o[d] = 0.0f;
    for (int64_t j = offsets[b]; j < offsets[b + 1]; ++j) {
      const float* x = table + idx_at(ids, idx64, j) * dim;
      for (int64_t d = 0; d < dim; ++d) o[d] += x[d];
    }
    int64_t cnt = offsets[b + 1] - offsets[b];
    if (combiner == 1 && cnt > 0) {
      const float inv = 1.0f / (float)(int32_t)cnt;
      for (int64_t d = 0; d < dim; ++d) o[d] *= inv;
    }
  }
}

/* ======================================================================== */
/* __pooling (annc/service/cpu/graph_opt.cc:131-176).                       */
/* ======================================================================== */
/* KPFusedSparseSegmentReduceNonzero
 * (annc/tensorflow/kernels/embedding_fused_sparse_segment_reduce_nonzero.cc:39-372):
 * segments in order of first appearance (:86-113), rows added in index order
 * per dim, mean = sum * (1/count), values != 0 listed with their (segment) or
 * (segment, dim) coordinates; shape = max(0, max segment id) + 1 (:62-71).
 * Writes at most cap values; returns their total number. */
int64_t ora_segment_reduce_nonzero(const float* data, int64_t rows, int64_t dim,
                                   const void* indices, int idx64, const int64_t* seg,
                                   int64_t seg_stride, int64_t n, int combiner, int one_d,
                                   int32_t* out_shape, int32_t* out_idx, float* out_val,
                                   int64_t cap) {
  (void)rows;
  int64_t max_seg = 0, nseg = 0;
  int64_t* order = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n > 0 ? n : 1));
  float* sums = (float*)calloc((size_t)(n > 0 ? n : 1) * (size_t)(dim > 0 ? dim : 1), sizeof(float));
  int32_t* counts = (int32_t*)calloc((size_t)(n > 0 ? n : 1), sizeof(int32_t));
  for (int64_t i = 0; i < n; ++i) {
    const int64_t s = seg[i * seg_stride];
    if (s > max_seg) max_seg = s;
    int64_t k = 0;
    while (k < nseg && order[k] != s) ++k;
    if (k == nseg) order[nseg++] = s;
    const int64_t row = idx64 ? ((const int64_t*)indices)[i] : ((const int32_t*)indices)[i];
    for (int64_t d = 0; d < dim; ++d) sums[k * dim + d] += data[row * dim + d];
    counts[k]++;
  }
  out_shape[0] = (int32_t)(max_seg + 1);
  if (!one_d) out_shape[1] = (int32_t)dim;
  int64_t nz = 0;
  for (int64_t k = 0; k < nseg; ++k) {
    const float inv = combiner == 1 ? (counts[k] > 0 ? 1.0f / (float)counts[k] : 0.0f) : 1.0f;
    for (int64_t d = 0; d < dim; ++d) {
      const float v = sums[k * dim + d] * inv;
      if (v != 0.0f) {
        if (nz < cap) {
          if (one_d) {
            out_idx[nz] = (int32_t)order[k];
          } else {
            out_idx[2 * nz] = (int32_t)order[k];
            out_idx[2 * nz + 1] = (int32_t)d;
          }
          out_val[nz] = v;
        }
        ++nz;
      }
    }
  }
  free(order);
  free(sums);
  free(counts);
  return nz;
}

void ora_pooling(const int64_t* ids, const float* gathered, int64_t m, int64_t k, int64_t n,
                 const int64_t* ss, const int64_t* sl, float* out) {
  for (int64_t i = 0; i < m; ++i) {
    float red = 0.0f;
    for (int64_t j = 0; j < k; ++j) red += (float)(ids[i * k + j] > 0);
    const int empty = (red == 0.0f);
    for (int64_t p = 0; p < n; ++p) {
      float sum = 0.0f;
      for (int64_t j = 0; j < k; ++j) {
        float v = 0.0f;
        if (i >= ss[0] && i < sl[0] && j >= ss[1] && j < sl[1] && p >= ss[2] && p < sl[2] &&
            ids[i * k + j] > 0)
          v = gathered[i * k * n + j * n + p];
        sum += v;
      }
      out[i * n + p] = empty ? 0.0f : sum / red;
    }
  }
}

/* __reduce_mean (annc/service/cpu/reduce_rewriter.cc:31-46): out[i] =
 * sasum of the i-th run of m values, divided by (int)m. */
void ora_reduce_mean(const float* x, int64_t m, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    float s = 0.0f;
    for (int64_t j = 0; j < m; ++j) s += fabsf(x[i * m + j]);
    out[i] = s / (float)(int)m;
  }
}

/* sparse_embedding2 (graph_opt.cc:8-41; bounds from
 * bisheng-cpu/embedding_simplify.cc:62-81):
 * out[i,:] = table[valid ? id : fallback, :] * (float)valid. */
/* KPFusedGather (annc/tensorflow/kernels/embedding_fused_gather.cc:48-84):
 * walk the key column in row order with a map key -> first-occurrence index
 * (open addressing here, unordered_map there); a new key gets the next index
 * and joins `unique`; every row records its key's index.  Then the table
 * rows of the unique keys are copied.  Returns the unique count, or -1 if a
 * unique key lies outside [0, rows) ("idx out of table range"). */
int64_t ora_fused_gather(const float* table, int64_t rows, int64_t dim, const int64_t* keys,
                         int64_t stride, int64_t n, int64_t* unique, int32_t* indices,
                         float* out) {
  int64_t cap = 16;
  while (cap < 2 * n) cap <<= 1;
  int64_t* slot_key = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  int32_t* slot_idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)cap);
  for (int64_t i = 0; i < cap; ++i) slot_idx[i] = -1;
  int64_t u = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t key = keys[i * stride];
    uint64_t h = (uint64_t)key * 0x9e3779b97f4a7c15ULL;
    int64_t at = (int64_t)(h >> 17) & (cap - 1);
    while (slot_idx[at] >= 0 && slot_key[at] != key) at = (at + 1) & (cap - 1);
    if (slot_idx[at] < 0) {
      slot_key[at] = key;
      slot_idx[at] = (int32_t)u;
      unique[u++] = key;
    }
    indices[i] = slot_idx[at];
  }
  free(slot_key);
  free(slot_idx);
  for (int64_t r = 0; r < u; ++r) {
    if (unique[r] < 0 || unique[r] >= rows) return -1;
    memcpy(out + r * dim, table + unique[r] * dim, sizeof(float) * (size_t)dim);
  }
  return u;
}

/* KPFusedBatchMatMulAddSigmoid, the generic path
 * (annc/tensorflow/kernels/fused_batchmatmul_add_sigmoid.cc ComputeGeneric,
 * with the bias broadcast of BuildBiasInfo): acc = bias, acc += lhs * rhs in
 * k order, out = 1 / (1 + exp(-acc)) (the reference test's Sigmoid).
 * bias_dims holds the right-aligned [3] dims, each 1 or full. */
void ora_batch_matmul_add_sigmoid(const float* lhs, const float* rhs, int rhs_batched,
                                  const float* bias, const int64_t* bias_dims, int64_t batch,
                                  int64_t m, int64_t k, int64_t n, float* out) {
  const int64_t s2 = bias_dims[2] == 1 ? 0 : 1;
  const int64_t s1 = bias_dims[1] == 1 ? 0 : bias_dims[2];
  const int64_t s0 = bias_dims[0] == 1 ? 0 : bias_dims[1] * bias_dims[2];
  for (int64_t b = 0; b < batch; ++b) {
    const float* lb = lhs + b * m * k;
    const float* rb = rhs + (rhs_batched ? b * k * n : 0);
    for (int64_t i = 0; i < m; ++i) {
      for (int64_t j = 0; j < n; ++j) {
        float acc = bias[b * s0 + i * s1 + j * s2];
        for (int64_t kk = 0; kk < k; ++kk) acc += lb[i * k + kk] * rb[kk * n + j];
        out[(b * m + i) * n + j] = 1.0f / (1.0f + expf(-acc));
      }
    }
  }
}

void ora_sparse_embedding2(const float* table, int64_t rows, int64_t dim, const void* ids,
                           int idx64, int64_t n, int64_t fallback, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t id = idx_at(ids, idx64, i);
    int valid = (id >= 0) && (id < rows);
    const float* x = table + (valid ? id : fallback) * dim;
    const float mask = (float)valid;
    for (int64_t d = 0; d < dim; ++d) out[i * dim + d] = x[d] * mask;
  }
}

/* ======================================================================== */
/* Hash-bucket embedding ops                                                 */
/* ======================================================================== */
/* KPFusedEmbeddingWithHashBucketOp::Compute
 * (python/tensorflow/kernels/fused_embedding_with_hash_bucket.cc:49-76). */
void ora_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets, int64_t batch,
                                    const float* weight, int64_t dim, int64_t num_buckets,
                                    float* out) {
  memset(out, 0, sizeof(float) * (size_t)(batch * dim));
  for (int64_t i = 0; i < batch; ++i) {
    int64_t len = offsets[i + 1] - offsets[i];
    if (len == 0) continue;
    uint64_t x = ora_fingerprint64(bytes + offsets[i], (size_t)len) % (uint64_t)num_buckets;
    memcpy(out + i * dim, weight + x * dim, sizeof(float) * (size_t)dim);
  }
}

/* KPFusedDnnEmbeddingWithHashBucketOp / KPFusedLinearEmbeddingWithHashBucketOp
 * (fused_dnn_embedding_with_hash_bucket.cc:19-46). */
void ora_dnn_embedding_with_hash_bucket(const char* bytes, const int64_t* offsets, int64_t batch,
                                        const float* weight, int64_t rows, int64_t dim,
                                        int64_t num_buckets, float* out) {
  memset(out, 0, sizeof(float) * (size_t)(batch * dim));
  for (int64_t i = 0; i < batch; ++i) {
    const char* p = bytes + offsets[i];
    int64_t span = offsets[i + 1] - offsets[i];
    if (span == 0) continue; /* input(i) != "" compares the whole string */
    uint64_t h = ora_fingerprint64(p, str_len(p, span, 1));
    int64_t b = (int64_t)(h % (uint64_t)num_buckets);
    if (b >= 0 && b < rows) memcpy(out + i * dim, weight + b * dim, sizeof(float) * (size_t)dim);
  }
}

/* KPFusedSparseEmbeddingOp::Compute (fused_sparse_embedding.cc:25-84). */
void ora_sparse_embedding(const char* bytes, const int64_t* offsets, int64_t n,
                          int64_t num_buckets, int64_t* indices, int64_t* values,
                          uint8_t* empty, int64_t* shape, int64_t* num_values) {
  int64_t nv = 0;
  for (int64_t i = 0; i < n; ++i) {
    const char* p = bytes + offsets[i];
    int64_t span = offsets[i + 1] - offsets[i];
    indices[2 * i] = i;
    indices[2 * i + 1] = 0;
    if (span > 0) {
      uint64_t h = ora_fingerprint64(p, str_len(p, span, 1));
      int64_t x = (int64_t)(h % (uint64_t)num_buckets);
      if (x > 0) {
        values[nv] = x;
        empty[nv] = 0;
        ++nv;
      }
    } else {
      values[nv] = 0;
      empty[nv] = 1;
      ++nv;
    }
  }
  shape[0] = n;
  shape[1] = 1;
  *num_values = nv;
}

/* Multi-field hashed bags: AsString -> Fingerprint64 -> % buckets -> the
 * segment-reduce order above, written into out[b, f*dim ..]. */
void ora_hashed_embedding_bags(int64_t nfields, int64_t batch, int64_t dim,
                               const float* const* tables, const int64_t* num_buckets,
                               const int64_t* ids, const int64_t* offsets, int combiner,
                               float* out, int64_t ldo, int64_t* buckets_out, int nthreads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#else
  (void)nthreads;
#endif
  for (int64_t bag = 0; bag < nfields * batch; ++bag) {
    int64_t f = bag / batch, b = bag % batch;
    float* o = out + b * ldo + f * dim;
    char buf[32];
    for (int64_t d = 0; d < dim; ++d) o[d] = 0.0f;
    for (int64_t j = offsets[bag]; j < offsets[bag + 1]; ++j) {
      int len = ora_format_int64(ids[j], buf);
      int64_t bk = (int64_t)(ora_fingerprint64(buf, (size_t)len) % (uint64_t)num_buckets[f]);
      if (buckets_out) buckets_out[j] = bk;
      const float* x = tables[f] + bk * dim;
      for (int64_t d = 0; d < dim; ++d) o[d] += x[d];
    }
    int64_t cnt = offsets[bag + 1] - offsets[bag];
    if (combiner == 1 && cnt > 0) {
      const float inv = 1.0f / (float)(int32_t)cnt;
      for (int64_t d = 0; d < dim; ++d) o[d] *= inv;
    }
  }
}

/* ======================================================================== */
/* GEMM custom calls over OpenBLAS sgemm (gemm_rewriter.cc:136-281).         */
/* The reference links OpenBLAS 0.3.29 (third_party/repo.bzl:7); the same    */
/* release ships with numpy as scipy_openblas64_ (64-bit integer ABI).      */
/* ======================================================================== */
typedef void (*sgemm64_fn)(int order, int ta, int tb, int64_t m, int64_t n, int64_t k,
                           float alpha, const float* a, int64_t lda, const float* b,
                           int64_t ldb, float beta, float* c, int64_t ldc);
typedef void (*set_threads_fn)(int n);
typedef char* (*get_config_fn)(void);
static sgemm64_fn g_sgemm = NULL;
static set_threads_fn g_set_threads = NULL;
static get_config_fn g_get_config = NULL;

enum { kRowMajor = 101, kNoTrans = 111 };

/* Loads the OpenBLAS library at `path`; returns 0 on success. */
int ora_blas_load(const char* path) {
  void* h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!h) return -1;
  g_sgemm = (sgemm64_fn)dlsym(h, "scipy_cblas_sgemm64_");
  g_set_threads = (set_threads_fn)dlsym(h, "scipy_openblas_set_num_threads64_");
  g_get_config = (get_config_fn)dlsym(h, "scipy_openblas_get_config64_");
  return g_sgemm ? 0 : -2;
}

const char* ora_blas_config(void) { return g_get_config ? g_get_config() : "unloaded"; }

void ora_blas_set_threads(int n) {
  if (g_set_threads) g_set_threads(n);
}

int ora_sgemm(int64_t m, int64_t n, int64_t k, float alpha, const float* a, int64_t lda,
              const float* b, int64_t ldb, float beta, float* c, int64_t ldc) {
  if (!g_sgemm) return -1;
  g_sgemm(kRowMajor, kNoTrans, kNoTrans, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc);
  return 0;
}

/* __matmul: C = A.B (gemm_rewriter.cc:161-185). */
int ora_matmul(int64_t m, int64_t n, int64_t k, const float* a, const float* b, float* c) {
  return ora_sgemm(m, n, k, 1.0f, a, k, b, n, 0.0f, c, n);
}

/* __matmul_add: memcpy E then sgemm beta=1 (gemm_rewriter.cc:218-247). */
int ora_matmul_add(int64_t m, int64_t n, int64_t k, const float* e, const float* a,
                   const float* b, float* c) {
  memcpy(c, e, sizeof(float) * (size_t)(m * n));
  return ora_sgemm(m, n, k, 1.0f, a, k, b, n, 1.0f, c, n);
}

/* __matmul_add_relu: as above then std::max(x, 0.f) (gemm_rewriter.cc:249-281). */
int ora_matmul_add_relu(int64_t m, int64_t n, int64_t k, const float* e, const float* a,
                        const float* b, float* c) {
  int rc = ora_matmul_add(m, n, k, e, a, b, c);
  for (int64_t i = 0; i < m * n; ++i) c[i] = (c[i] < 0.0f) ? 0.0f : c[i];
  return rc;
}

/* __batch_matmul: loop of sgemms (gemm_rewriter.cc:187-216). */
int ora_batch_matmul(int64_t batch, int64_t m, int64_t n, int64_t k, const float* a,
                     const float* b, float* c) {
  for (int64_t i = 0; i < batch; ++i) {
    int rc = ora_sgemm(m, n, k, 1.0f, a + i * m * k, k, b + i * k * n, n, 0.0f, c + i * m * n, n);
    if (rc) return rc;
  }
  return 0;
}

/* Dense layer as the reference graph runs it around __layout_matmul /
 * __matmul_add_relu: sgemm, then bias broadcast-add, then the activation
 * (0 none, 1 relu, 2 sigmoid) as separate loops. */
int ora_dense_layer(int64_t m, int64_t n, int64_t k, const float* a, int64_t lda,
                    const float* w, const float* bias, int act, float* c) {
  int rc = ora_sgemm(m, n, k, 1.0f, a, lda, w, n, 0.0f, c, n);
  for (int64_t i = 0; i < m; ++i) {
    float* row = c + i * n;
    if (bias)
      for (int64_t j = 0; j < n; ++j) row[j] += bias[j];
    if (act == 1)
      for (int64_t j = 0; j < n; ++j) row[j] = (row[j] < 0.0f) ? 0.0f : row[j];
    else if (act == 2)
      for (int64_t j = 0; j < n; ++j) row[j] = 1.0f / (1.0f + expf(-row[j]));
  }
  return rc;
}
