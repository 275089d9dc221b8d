// probe.hip -- measurement kernel: steady-state random row gathers.
//
// Not an operator.  It reads rows at uniformly random positions of a table,
// U rows in flight per group of G lanes (a row of 4G floats, one 16-byte
// load per lane), with no dependent index loads, so it measures the rate at
// which gfx950 serves random row reads (each a whole 128-byte line from the
// fabric for rows of up to 128 bytes) when nothing else limits the kernel:
// the ceiling against which the embedding-bag kernels' random gathers are
// compared.  Every thread writes one sum, so no load is dead.
//
// Built into its own library, libannc_probe.so (bench.py loads it), and not
// part of the operator library or its header.  Returns 0, or 3 for
// arguments it refuses, or 13 when the launch fails.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace annc {
namespace {

constexpr int kThreads = 256;

template <int G, int U>
__global__ __launch_bounds__(kThreads) void probe_random_rows_kernel(const float* __restrict__ table,
                                                                      uint32_t rows, int iters,
                                                                      float* __restrict__ out) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int grp = threadIdx.x / G, l = threadIdx.x % G;
  // one linear congruential stream per lane group (Numerical Recipes'
  // 32-bit constants), seeded by the group's global number
  uint32_t x = (blockIdx.x * (kThreads / G) + grp) * 2654435761u + 12345u;
  f32x4 acc = f32x4(0.0f);
  const f32x4* t4 = reinterpret_cast<const f32x4*>(table);
  for (int it = 0; it < iters; it += U) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      x = x * 1664525u + 1013904223u;
      const uint32_t row = x % rows;
      v[u] = t4[static_cast<int64_t>(row) * G + l];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u];
  }
  out[static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x] = acc.x + acc.y + acc.z + acc.w;
}

}  // namespace
}  // namespace annc

extern "C" int annc_probe_random_rows(void* stream, const float* table, int64_t rows,
                                      int64_t dim, int64_t blocks, int64_t rows_per_group,
                                      float* out) {
  using namespace annc;
  if (!table || !out) return 3;
  if (rows < 1 || rows >= (int64_t(1) << 32)) return 3;
  if (dim != 16 && dim != 32 && dim != 64) return 3;
  if (blocks < 1 || blocks >= (int64_t(1) << 31)) return 3;
  if (rows_per_group < 8 || rows_per_group % 8 != 0 || rows_per_group >= (1 << 30)) return 3;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int iters = static_cast<int>(rows_per_group);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, table,
                       static_cast<uint32_t>(rows), iters, out);
  };
  if (dim == 16)
    go(probe_random_rows_kernel<4, 8>);
  else if (dim == 32)
    go(probe_random_rows_kernel<8, 8>);
  else
    go(probe_random_rows_kernel<16, 8>);
  return hipGetLastError() == hipSuccess ? 0 : 13;
}
