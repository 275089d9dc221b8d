// custom_calls.cpp -- the XLA-CPU custom-call targets of ANNC's GEMM path.
//
// Same symbol names, operand order and shape-info operands as the reference
// (annc/service/cpu/gemm_rewriter.cc:136-281, graph_opt.cc:131-176,
// registration list kdnn_rewriter.h:148-155).  Operands may be host memory
// (XLA-CPU buffers: staged through the device on the library stream) or
// device memory (used in place); the call returns when `out` holds the
// result.  The XLA ABI has no error channel: failures are recorded in
// annc_hip_last_error() and reported once on stderr, leaving `out` unwritten.
#include <atomic>
#include <cstdio>
#include <cstring>

#include "common.h"
#include "embedding_impl.h"

namespace annc {
namespace {

std::atomic<bool> g_reported{false};

void report(const char* target, int rc) {
  if (rc == ANNC_OK) {
    clear_error();
    return;
  }
  if (!g_reported.exchange(true))
    std::fprintf(stderr, "[ANNC ERROR] %s: %s\n", target, annc_hip_last_error());
}

struct GemmCall {
  const void* a;
  const void* b;
  const void* e;
  const int64_t* shape_a;  // s64[2*rank] dims..., minor_to_major...
  const int64_t* shape_b;
  int rank;
  bool packed;
};

int run_gemm(void* out, const GemmCall& g) {
  int64_t sa[6] = {0}, sb[6] = {0};
  int rc = read_i64(g.shape_a, 2 * g.rank, sa);
  if (rc == ANNC_OK) rc = read_i64(g.shape_b, 2 * g.rank, sb);
  if (rc != ANNC_OK) return rc;
  int64_t batch = 1, m, k, n;
  if (g.rank == 3) {
    batch = sa[0];
    m = sa[1];
    k = sa[2];
    n = sb[2];
  } else {
    m = sa[0];
    k = sa[1];
    n = sb[1];
  }
  ANNC_REQUIRE(batch >= 0 && m >= 0 && k >= 0 && n >= 0, "negative dimension in shape info");
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const size_t fa = sizeof(float);
  const float* A = static_cast<const float*>(st.in(g.a, fa * batch * m * k));
  const float* B = static_cast<const float*>(st.in(g.b, fa * batch * k * n));
  const float* E = static_cast<const float*>(st.in(g.e, fa * m * n));
  float* C = static_cast<float*>(st.out(out, fa * batch * m * n));
  if (st.status() != ANNC_OK) return st.status();
  rc = annc_hip_gemm(s, batch, m, n, k, A, k, m * k, B, n, k * n, g.packed ? 1 : 0, E, n, 0,
                     nullptr, 0, C, n, m * n);
  if (rc != ANNC_OK) return rc;
  return st.finish();
}

int run_gemm_relu(void* out, const GemmCall& g) {
  // Same as run_gemm with the ReLU epilogue (gemm_rewriter.cc:278-280).
  int64_t sa[4], sb[4];
  int rc = read_i64(g.shape_a, 4, sa);
  if (rc == ANNC_OK) rc = read_i64(g.shape_b, 4, sb);
  if (rc != ANNC_OK) return rc;
  const int64_t m = sa[0], k = sa[1], n = sb[1];
  ANNC_REQUIRE(m >= 0 && k >= 0 && n >= 0, "negative dimension in shape info");
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const size_t fa = sizeof(float);
  const float* A = static_cast<const float*>(st.in(g.a, fa * m * k));
  const float* B = static_cast<const float*>(st.in(g.b, fa * k * n));
  const float* E = static_cast<const float*>(st.in(g.e, fa * m * n));
  float* C = static_cast<float*>(st.out(out, fa * m * n));
  if (st.status() != ANNC_OK) return st.status();
  rc = annc_hip_gemm(s, 1, m, n, k, A, k, 0, B, n, 0, 0, E, n, 0, nullptr, ANNC_EPI_RELU, C, n, 0);
  if (rc != ANNC_OK) return rc;
  return st.finish();
}

int run_pooling(void* out, void** in) {
  int64_t ids_shape[4], g_shape[6], ss[3], sl[3];
  int rc = read_i64(in[4], 4, ids_shape);
  if (rc == ANNC_OK) rc = read_i64(in[5], 6, g_shape);
  if (rc == ANNC_OK) rc = read_i64(in[2], 3, ss);
  if (rc == ANNC_OK) rc = read_i64(in[3], 3, sl);
  if (rc != ANNC_OK) return rc;
  const int64_t m = ids_shape[0], k = ids_shape[1], n = g_shape[2];
  ANNC_REQUIRE(m >= 0 && k >= 0 && n >= 0, "negative dimension in shape info");
  const int64_t dims[3] = {m, k, n};
  for (int d = 0; d < 3; ++d)
    ANNC_REQUIRE(ss[d] >= 0 && ss[d] <= sl[d] && sl[d] <= dims[d],
                 "__pooling slice [%lld, %lld) outside dimension %d of size %lld",
                 (long long)ss[d], (long long)sl[d], d, (long long)dims[d]);
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const int64_t* ids = static_cast<const int64_t*>(st.in(in[0], sizeof(int64_t) * m * k));
  const float* gathered = static_cast<const float*>(st.in(in[1], sizeof(float) * m * k * n));
  float* o = static_cast<float*>(st.out(out, sizeof(float) * m * n));
  if (st.status() != ANNC_OK) return st.status();
  rc = annc_hip_pooling(s, ids, gathered, m, k, n, ss, sl, o);
  if (rc != ANNC_OK) return rc;
  return st.finish();
}

int run_reduce_mean(void* out, const void** in) {
  // reduce_rewriter.cc:31-46: in[0] (the axis, read as a float) is unused;
  // in[1] holds n runs of m values, m = shape[0] and n = shape[1] of in[3].
  int64_t shape[2];
  const int rc0 = read_i64(in[3], 2, shape);
  if (rc0 != ANNC_OK) return rc0;
  const int64_t m = shape[0], n = shape[1];
  ANNC_REQUIRE(m >= 0 && n >= 0, "negative dimension in shape info");
  if (n == 0) return ANNC_OK;
  hipStream_t s = lib_stream();
  if (!s) return set_error(ANNC_INTERNAL, "no HIP stream");
  Staging st(s);
  const float* x = static_cast<const float*>(st.in(in[1], sizeof(float) * (size_t)(m * n)));
  float* o = static_cast<float*>(st.out(out, sizeof(float) * (size_t)n));
  if (st.status() != ANNC_OK) return st.status();
  const int rc = launch_abs_mean(s, x, m, n, o);
  if (rc != ANNC_OK) return rc;
  return st.finish();
}

struct Target {
  const char* name;
  void* fn;
};

}  // namespace
}  // namespace annc

extern "C" {

void __matmul(void* out, const void** in) {
  annc::GemmCall g{in[0], in[1], nullptr, static_cast<const int64_t*>(in[2]),
                   static_cast<const int64_t*>(in[3]), 2, false};
  annc::report("__matmul", annc::run_gemm(out, g));
}

void __matmul_add(void* out, const void** in) {
  annc::GemmCall g{in[1], in[2], in[0], static_cast<const int64_t*>(in[4]),
                   static_cast<const int64_t*>(in[5]), 2, false};
  annc::report("__matmul_add", annc::run_gemm(out, g));
}

void __matmul_add_relu(void* out, const void** in) {
  // in[0] is the broadcast zero of max(); like the reference it is unused.
  annc::GemmCall g{in[2], in[3], in[1], static_cast<const int64_t*>(in[6]),
                   static_cast<const int64_t*>(in[7]), 2, false};
  annc::report("__matmul_add_relu", annc::run_gemm_relu(out, g));
}

void __batch_matmul(void* out, const void** in) {
  annc::GemmCall g{in[0], in[1], nullptr, static_cast<const int64_t*>(in[2]),
                   static_cast<const int64_t*>(in[3]), 3, false};
  annc::report("__batch_matmul", annc::run_gemm(out, g));
}

void __layout_matmul(void* out, const void** in) {
  annc::GemmCall g{in[0], in[1], nullptr, static_cast<const int64_t*>(in[2]),
                   static_cast<const int64_t*>(in[3]), 2, true};
  annc::report("__layout_matmul", annc::run_gemm(out, g));
}

void __pooling(void* out, void** in) { annc::report("__pooling", annc::run_pooling(out, in)); }

void __reduce_mean(void* out, const void** in) {
  annc::report("__reduce_mean", annc::run_reduce_mean(out, in));
}

static const annc::Target kTargets[] = {
    {"__matmul", reinterpret_cast<void*>(&__matmul)},
    {"__batch_matmul", reinterpret_cast<void*>(&__batch_matmul)},
    {"__matmul_add", reinterpret_cast<void*>(&__matmul_add)},
    {"__matmul_add_relu", reinterpret_cast<void*>(&__matmul_add_relu)},
    {"__reduce_mean", reinterpret_cast<void*>(&__reduce_mean)},
    {"__pooling", reinterpret_cast<void*>(&__pooling)},
    {"__layout_matmul", reinterpret_cast<void*>(&__layout_matmul)},
};

void* annc_custom_call_target(const char* name) {
  if (!name) return nullptr;
  for (const annc::Target& t : kTargets)
    if (std::strcmp(t.name, name) == 0) return t.fn;
  return nullptr;
}

int annc_register_custom_call_targets(void (*cb)(const char*, void*, void*), void* user) {
  int count = 0;
  for (const annc::Target& t : kTargets) {
    if (cb) cb(t.name, t.fn, user);
    ++count;
  }
  return count;
}

}  // extern "C"
