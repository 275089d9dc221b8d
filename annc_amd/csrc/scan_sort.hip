// scan_sort.hip -- device-wide prefix sums and a stable LSD radix sort of
// (uint32 key, int32 value) pairs, for the segment-reduction and compaction
// paths of the embedding ops:
//   * KPFusedSparseSegmentReduce with more segment ids than the counting
//     sort covers (embedding_fused_sparse_segment_reduce.cc:92-131): a
//     stable sort of positions by segment id, so each segment's rows are
//     still added in position order;
//   * KPFusedSparseEmbedding's compaction of kept ids
//     (python/tensorflow/kernels/fused_sparse_embedding.cc:25-84) and the
//     nonzero listing of KPFusedSparseSegmentReduceNonzero: an exclusive or
//     inclusive sum of 0/1 flags.
//
// Scan (n values, tiles of kScanTile = 4096):
//   1. scan_tile_sum_kernel   one workgroup per tile: the tile's total;
//   2. scan_totals_kernel     one 1024-thread workgroup: exclusive prefix of
//                             the tile totals, in place;
//   3. scan_tile_kernel       one workgroup per tile: the tile is staged in
//                             LDS with coalesced loads, each thread sums 16
//                             consecutive values, the 256 thread sums are
//                             scanned by wave shuffles and LDS, and the
//                             results go back through LDS, coalesced.
// Radix sort (8-bit digits, ceil(end_bit / 8) passes, blocks of kRsBlock):
//   1. rs_hist_kernel    per block: digit counts, stored digit-major as
//                        H[digit * blocks + block];
//   2. the scan above    exclusive prefix of H: where each (digit, block)
//                        run starts in the output;
//   3. rs_scatter_kernel per block: each of the 4 waves walks its quarter
//                        of the block in order, 64 positions at a time;
//                        lanes with the same digit rank themselves by lane
//                        order (ballots over the 8 digit bits), so equal
//                        digits keep their order: every pass is stable.
// Integer work only: results do not depend on timing or launch shape.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "common.h"
#include "scan_sort.h"

namespace annc {
namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;
constexpr int kTotalsThreads = 1024;

constexpr int kRsThreads = 256;
constexpr int kRsWaves = kRsThreads / 64;
constexpr int kRsChunk = 1024;                  // positions per wave
constexpr int kRsBlock = kRsWaves * kRsChunk;   // positions per workgroup
constexpr int kRsBins = 256;

size_t round256(size_t x) { return (x + 255) & ~size_t(255); }

__device__ __forceinline__ int wave_inclusive_sum(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d);
    if (lane >= d) v += u;
  }
  return v;
}

// Exclusive prefix over the workgroup (blockDim.x threads, up to 1024) of
// one int per thread; *total receives the sum.  `lds` holds 16 ints.
__device__ __forceinline__ int block_exclusive_sum(int v, int* lds, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int waves = (blockDim.x + 63) >> 6;
  const int incl = wave_inclusive_sum(v);
  if (lane == 63) lds[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < waves; ++w) {
    const int t = lds[w];
    before += w < wave ? t : 0;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + incl - v;
}

template <typename T>
__global__ __launch_bounds__(kScanThreads) void scan_tile_sum_kernel(const T* __restrict__ in,
                                                                     int64_t n,
                                                                     int* __restrict__ sums) {
  __shared__ int lds[16];
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  int v = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    const int64_t i = base + j * kScanThreads + threadIdx.x;
    if (i < n) v += static_cast<int>(in[i]);
  }
  int total;
  block_exclusive_sum(v, lds, &total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Exclusive prefix of sums[0..t) in place; sums[t] receives the total.
__global__ __launch_bounds__(kTotalsThreads) void scan_totals_kernel(int* __restrict__ sums,
                                                                     int64_t t) {
  __shared__ int lds[16];
  const int64_t per = (t + kTotalsThreads - 1) / kTotalsThreads;
  const int64_t b = per * threadIdx.x, e = std::min<int64_t>(b + per, t);
  int v = 0;
  for (int64_t i = b; i < e; ++i) v += sums[i];
  int total;
  int run = block_exclusive_sum(v, lds, &total);
  for (int64_t i = b; i < e; ++i) {
    const int x = sums[i];
    sums[i] = run;
    run += x;
  }
  if (threadIdx.x == 0) sums[t] = total;
}

template <typename T, bool INCLUSIVE>
__global__ __launch_bounds__(kScanThreads) void scan_tile_kernel(const T* __restrict__ in,
                                                                 int64_t n,
                                                                 const int* __restrict__ sums,
                                                                 T* __restrict__ out) {
  // +1 int per 16 so a thread's 16 consecutive values sit in distinct banks
  __shared__ int tile[kScanTile + kScanTile / 16];
  __shared__ int lds[16];
  auto at = [](int i) { return i + (i >> 4); };
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    const int c = j * kScanThreads + threadIdx.x;
    const int64_t i = base + c;
    tile[at(c)] = i < n ? static_cast<int>(in[i]) : 0;
  }
  __syncthreads();
  const int c0 = threadIdx.x * kScanItems;
  int v = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) v += tile[at(c0 + j)];
  int total;
  int run = block_exclusive_sum(v, lds, &total) + sums[blockIdx.x];
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    const int x = tile[at(c0 + j)];
    tile[at(c0 + j)] = INCLUSIVE ? run + x : run;
    run += x;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    const int c = j * kScanThreads + threadIdx.x;
    const int64_t i = base + c;
    if (i < n) out[i] = static_cast<T>(tile[at(c)]);
  }
}

template <typename T>
int scan_impl(hipStream_t s, const T* in, T* out, int64_t n, bool inclusive, void* temp) {
  ANNC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "scan length out of range");
  if (n == 0) return ANNC_OK;
  const int64_t tiles = (n + kScanTile - 1) / kScanTile;
  int* sums = static_cast<int*>(temp);
  hipLaunchKernelGGL(scan_tile_sum_kernel<T>, dim3((unsigned)tiles), dim3(kScanThreads), 0, s, in,
                     n, sums);
  ANNC_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(scan_totals_kernel, dim3(1), dim3(kTotalsThreads), 0, s, sums, tiles);
  ANNC_HIP_TRY(hipGetLastError());
  if (inclusive)
    hipLaunchKernelGGL((scan_tile_kernel<T, true>), dim3((unsigned)tiles), dim3(kScanThreads), 0,
                       s, in, n, sums, out);
  else
    hipLaunchKernelGGL((scan_tile_kernel<T, false>), dim3((unsigned)tiles), dim3(kScanThreads), 0,
                       s, in, n, sums, out);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

__global__ __launch_bounds__(kRsThreads) void rs_hist_kernel(const uint32_t* __restrict__ keys,
                                                             int64_t n, int shift, int64_t blocks,
                                                             uint32_t* __restrict__ hist) {
  __shared__ int cnt[kRsBins];
  cnt[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kRsBlock;
  for (int j = 0; j < kRsBlock / kRsThreads; ++j) {
    const int64_t i = base + j * kRsThreads + threadIdx.x;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & (kRsBins - 1)], 1);
  }
  __syncthreads();
  hist[(int64_t)threadIdx.x * blocks + blockIdx.x] = static_cast<uint32_t>(cnt[threadIdx.x]);
}

__global__ __launch_bounds__(kRsThreads) void rs_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const int32_t* __restrict__ vals_in, int64_t n,
    int shift, int64_t blocks, const uint32_t* __restrict__ starts,
    uint32_t* __restrict__ keys_out, int32_t* __restrict__ vals_out) {
  __shared__ int cnt[kRsWaves][kRsBins];
  __shared__ uint32_t next[kRsWaves][kRsBins];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int w = 0; w < kRsWaves; ++w) cnt[w][threadIdx.x] = 0;
  __syncthreads();
  const int64_t chunk = (int64_t)blockIdx.x * kRsBlock + (int64_t)wave * kRsChunk;
  for (int j = 0; j < kRsChunk / 64; ++j) {
    const int64_t i = chunk + j * 64 + lane;
    if (i < n) atomicAdd(&cnt[wave][(keys_in[i] >> shift) & (kRsBins - 1)], 1);
  }
  __syncthreads();
  {
    // digit d = threadIdx.x: output start of each wave's run of d
    const int d = threadIdx.x;
    uint32_t run = starts[(int64_t)d * blocks + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) {
      next[w][d] = run;
      run += static_cast<uint32_t>(cnt[w][d]);
    }
  }
  __syncthreads();
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int j = 0; j < kRsChunk / 64; ++j) {
    const int64_t i = chunk + j * 64 + lane;
    const bool valid = i < n;
    const uint32_t key = valid ? keys_in[i] : 0u;
    const int d = static_cast<int>((key >> shift) & (kRsBins - 1));
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t set = __ballot((d >> b) & 1);
      same &= ((d >> b) & 1) ? set : ~set;
    }
    if (valid) {
      const int rank = __popcll(same & below);
      const uint32_t dst = next[wave][d] + static_cast<uint32_t>(rank);
      keys_out[dst] = key;
      vals_out[dst] = vals_in[i];
      // the last lane of each digit advances the run past this step's lanes
      if (rank == __popcll(same) - 1) next[wave][d] = dst + 1;
    }
  }
}

}  // namespace

size_t scan_temp_bytes(int64_t n) {
  const int64_t tiles = std::max<int64_t>(1, (n + kScanTile - 1) / kScanTile);
  return round256(sizeof(int) * (size_t)(tiles + 1));
}

int exclusive_sum(hipStream_t s, const int32_t* in, int32_t* out, int64_t n, void* temp) {
  return scan_impl<int32_t>(s, in, out, n, false, temp);
}

int inclusive_sum(hipStream_t s, const int32_t* in, int32_t* out, int64_t n, void* temp) {
  return scan_impl<int32_t>(s, in, out, n, true, temp);
}

size_t radix_sort_temp_bytes(int64_t n) {
  const int64_t blocks = std::max<int64_t>(1, (n + kRsBlock - 1) / kRsBlock);
  const int64_t h = blocks * kRsBins;
  return 2 * round256(sizeof(uint32_t) * (size_t)h) + scan_temp_bytes(h);
}

int radix_sort_pairs(hipStream_t s, uint32_t** keys, uint32_t** keys_alt, int32_t** vals,
                     int32_t** vals_alt, int64_t n, int end_bit, void* temp) {
  ANNC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "sort length out of range");
  ANNC_REQUIRE(end_bit >= 0 && end_bit <= 32, "key bits out of range");
  if (n == 0) return ANNC_OK;
  const int64_t blocks = (n + kRsBlock - 1) / kRsBlock;
  const int64_t h = blocks * kRsBins;
  ANNC_REQUIRE(h < (int64_t(1) << 31), "sort length out of range");
  uint32_t* hist = static_cast<uint32_t*>(temp);
  uint32_t* starts = reinterpret_cast<uint32_t*>(static_cast<char*>(temp) +
                                                 round256(sizeof(uint32_t) * (size_t)h));
  void* scan_tmp = static_cast<char*>(temp) + 2 * round256(sizeof(uint32_t) * (size_t)h);
  for (int shift = 0; shift < end_bit; shift += 8) {
    hipLaunchKernelGGL(rs_hist_kernel, dim3((unsigned)blocks), dim3(kRsThreads), 0, s, *keys, n,
                       shift, blocks, hist);
    ANNC_HIP_TRY(hipGetLastError());
    const int rc = scan_impl<uint32_t>(s, hist, starts, h, false, scan_tmp);
    if (rc != ANNC_OK) return rc;
    hipLaunchKernelGGL(rs_scatter_kernel, dim3((unsigned)blocks), dim3(kRsThreads), 0, s, *keys,
                       *vals, n, shift, blocks, starts, *keys_alt, *vals_alt);
    ANNC_HIP_TRY(hipGetLastError());
    std::swap(*keys, *keys_alt);
    std::swap(*vals, *vals_alt);
  }
  return ANNC_OK;
}

}  // namespace annc
