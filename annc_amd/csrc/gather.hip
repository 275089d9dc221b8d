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
//   2. position i is a first occurrence iff its slot's minimum is i; the
//      first occurrences are numbered in position order (the reference's
//      order) by block-local ranks plus a prefix over the blocks' counts;
//   3. indices[i] = number of the first occurrence of i's key; that
//      occurrence also writes unique[number] = key, and its workgroup copies
//      the table row of the key (G lanes per row, 16-byte loads where the
//      rows allow).
// U, the number of unique keys, is only known on the device.
#include <hip/hip_runtime.h>

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

// Insert workgroups of 1024 threads over 2048 positions: a key that is
// frequent in the data costs one global atomic per 2048 positions, not per
// 256 (configs[2]'s ids: 42.5 -> 37.4 us for the whole unique + gather;
// 4096 positions, at half the workgroups, was slower again).
constexpr int kUgThreads = 1024;         // threads of an insert workgroup
constexpr int kUgBlock = 2048;           // positions per workgroup
constexpr int kUgLocal = 2 * kUgBlock;   // LDS table slots (+1 for the empty marker's value)
// Largest key count of the global table: capacity is the power of two at
// or above 2n, and slot numbers (the empty marker `cap` too) are int32.
constexpr int64_t kMaxUniqueKeys = int64_t(1) << 29;

// Slot of every position's key in the global table, whose slots keep their
// key's smallest position (open addressing, linear probing; capacity a
// power of two >= 2n, so at most half the slots fill and every probe
// sequence ends).  Each workgroup first de-duplicates its kUgBlock
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
  __shared__ int32_t llist[kUgBlock];  // used LDS slots
  __shared__ int lcount;
  constexpr int kPer = kUgBlock / kUgThreads;
  static_assert(kUgBlock <= 2 * kUgThreads, "at most two listed keys per thread");
  for (int l = threadIdx.x; l < kUgLocal; l += kUgThreads) lkey[l] = kEmpty;
  for (int l = threadIdx.x; l <= kUgLocal; l += kUgThreads) lfirst[l] = INT_MAX;
  if (threadIdx.x == 0) {
    lempty = 0;
    lcount = 0;
  }
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
  // List the used LDS slots (at most one per position, so at most two per
  // thread), then insert each listed key: a thread's two probe chains run
  // side by side, each step one CAS that returns the slot's key, and the
  // block minimum goes in with an atomicMin whose result nobody waits for.
  for (int l = threadIdx.x; l <= kUgLocal; l += kUgThreads) {
    const bool used = l < kUgLocal ? lkey[l] != kEmpty : lempty != 0;
    const uint64_t m = __ballot(used);
    int base = 0;
    if ((threadIdx.x & 63) == 0 && m) base = atomicAdd(&lcount, __popcll(m));
    base = __shfl(base, 0, 64);
    if (used)
      llist[base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0))] = l;
  }
  __syncthreads();
  const int cnt = lcount;
  int sl[2];
  int64_t hk[2], key2[2];
  bool pend[2];
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const int e = threadIdx.x + v * kUgThreads;
    sl[v] = e < cnt ? llist[e] : -1;
    pend[v] = sl[v] >= 0 && sl[v] < kUgLocal;
    key2[v] = pend[v] ? lkey[sl[v]] : kEmpty;
    hk[v] = pend[v] ? static_cast<int64_t>(mix64(static_cast<uint64_t>(key2[v])) &
                                           (uint64_t)(cap - 1))
                    : cap;  // the empty marker's value has the extra global slot
  }
  for (int64_t probe = 0; probe < cap && (pend[0] || pend[1]); ++probe) {
    int64_t seen[2];
#pragma unroll
    for (int v = 0; v < 2; ++v)
      seen[v] = pend[v] ? static_cast<int64_t>(atomicCAS(
                              reinterpret_cast<unsigned long long*>(tab_key + hk[v]),
                              static_cast<unsigned long long>(kEmpty),
                              static_cast<unsigned long long>(key2[v])))
                        : kEmpty;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      if (!pend[v]) continue;
      if (seen[v] == kEmpty || seen[v] == key2[v])
        pend[v] = false;
      else
        hk[v] = (hk[v] + 1) & (cap - 1);
    }
  }
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    if (sl[v] < 0) continue;
    if (pend[v]) {  // cap probes without a slot: reported, never hangs
      atomicOr(status, 2);
      hk[v] = cap;
    }
    atomicMin(tab_first + hk[v], lfirst[sl[v]]);
    lslot[sl[v]] = static_cast<int32_t>(hk[v]);
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t i = b0 + u * kUgThreads + threadIdx.x;
    if (i < n) slot_of[i] = lslot[local[u]];
  }
}

// ---------------------------------------------------------------------------
// Numbering first occurrences (both engines).  With f(i) the smallest
// position of i's key, position i is a first occurrence iff f(i) == i, and
// its key's number is the count of first occurrences at positions <= f(i).
//   fr_rank_kernel    per block of kFrBlock positions: f(i) for every
//                     position, the block-local inclusive rank of each first
//                     occurrence, the block's count;
//   fr_prefix_kernel  (beyond kFrLdsBlocks blocks only) exclusive prefix of
//                     the block counts, one workgroup;
//   fr_number_kernel  one position per thread: number = prefix[block(f)] +
//                     rank[f], giving the inverse index, the unique keys,
//                     their count and (with a table) the rows of the unique
//                     keys whose first occurrence is in the workgroup.
// Up to kFrLdsBlocks blocks each number workgroup forms the prefix of the
// counts it needs in LDS, so the chain is two launches; the row copy runs in
// n/256 workgroups spread over the chip.
// ---------------------------------------------------------------------------
constexpr int kFrThreads = 256;
constexpr int kFrItems = 2;
constexpr int kFrShift = 9;
constexpr int kFrBlock = 1 << kFrShift;  // kFrThreads * kFrItems positions
constexpr int kFrWaves = kFrThreads / 64;
constexpr int kFrLdsBlocks = 1024;      // prefix formed in LDS: n <= 2^19
static_assert(kFrBlock == kFrThreads * kFrItems, "block = threads x items");

// f(i) through the hash table: the slot's smallest position
struct FirstBySlot {
  const int32_t* slot_of;
  const int32_t* tab_first;
  __device__ int32_t operator()(int64_t i) const { return tab_first[slot_of[i]]; }
};
// f(i) through the directly indexed table of a small key range
struct FirstByKey {
  const int64_t* keys;
  int64_t stride, kmin;
  const int32_t* first;
  __device__ int32_t operator()(int64_t i) const { return first[keys[i * stride] - kmin]; }
};

// Inclusive sum over the workgroup of one value per thread; *total gets the
// workgroup's sum.  Uses wsum[kFrWaves]; ends with every wave past its reads.
__device__ __forceinline__ int32_t fr_block_scan(int32_t v, int32_t* wsum, int32_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int32_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t x = __shfl_up(incl, off, 64);
    if (lane >= off) incl += x;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int32_t before = 0, all = 0;
#pragma unroll
  for (int q = 0; q < kFrWaves; ++q) {
    before += q < w ? wsum[q] : 0;
    all += wsum[q];
  }
  __syncthreads();
  *total = all;
  return before + incl;
}

// fpos[i] = f(i) (fpos may be the slot_of array f reads: each thread reads
// its own positions before writing them); rank[i] = 1-based rank of i among
// its block's first occurrences (written at first occurrences only);
// count[b] = the block's first occurrences.
template <class F>
__global__ __launch_bounds__(kFrThreads) void fr_rank_kernel(F first_of, int64_t n,
                                                             int32_t* fpos,
                                                             int32_t* __restrict__ rank,
                                                             int32_t* __restrict__ count) {
  __shared__ int32_t wc[kFrItems][kFrWaves];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t b0 = (int64_t)blockIdx.x << kFrShift;
  int32_t f[kFrItems];
#pragma unroll
  for (int u = 0; u < kFrItems; ++u) {
    const int64_t i = b0 + u * kFrThreads + t;
    f[u] = i < n ? first_of(i) : -1;
  }
  bool mk[kFrItems];
  int rk[kFrItems];
#pragma unroll
  for (int u = 0; u < kFrItems; ++u) {
    const int64_t i = b0 + u * kFrThreads + t;
    mk[u] = i < n && f[u] == static_cast<int32_t>(i);
    const uint64_t m = __ballot(mk[u]);
    rk[u] = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
    if (lane == 0) wc[u][w] = __popcll(m);
  }
  __syncthreads();
  // ranks in position order: item u's positions follow all of item u-1's
  int32_t before = 0;
#pragma unroll
  for (int u = 0; u < kFrItems; ++u) {
    int32_t off = before;
#pragma unroll
    for (int q = 0; q < kFrWaves; ++q) off += q < w ? wc[u][q] : 0;
    const int64_t i = b0 + u * kFrThreads + t;
    if (i < n) {
      fpos[i] = f[u];
      if (mk[u]) rank[i] = off + rk[u] + 1;
    }
#pragma unroll
    for (int q = 0; q < kFrWaves; ++q) before += wc[u][q];
  }
  if (t == 0) count[blockIdx.x] = before;
}

// pre[b] = sum of count[0..b) over nblk blocks, one workgroup
__global__ __launch_bounds__(kFrThreads) void fr_prefix_kernel(const int32_t* __restrict__ count,
                                                               int64_t nblk,
                                                               int32_t* __restrict__ pre) {
  __shared__ int32_t wsum[kFrWaves];
  int32_t carry = 0;
  for (int64_t base = 0; base < nblk; base += kFrThreads) {
    const int64_t j = base + threadIdx.x;
    const int32_t v = j < nblk ? count[j] : 0;
    int32_t total;
    const int32_t incl = fr_block_scan(v, wsum, &total);
    if (j < nblk) pre[j] = carry + incl - v;
    carry += total;
  }
}

// Position i = workgroup * kFrThreads + thread: indices[i] = number(f(i)) -
// 1; at first occurrences unique[number - 1] = key; the thread of the last
// position writes num_unique; with dim > 0 the workgroup then copies the
// rows of its first occurrences' keys, g lanes per row (VEC floats per
// lane), keys outside the table giving a zero row and the status bit.
// GPRE: the prefix comes from fr_prefix_kernel instead of being formed here.
template <int VEC, bool GPRE>
__global__ __launch_bounds__(kFrThreads) void fr_number_kernel(
    const int64_t* __restrict__ keys, int64_t stride, int64_t n, const int32_t* __restrict__ fpos,
    const int32_t* __restrict__ rank, const int32_t* __restrict__ count,
    const int32_t* __restrict__ gpre, int32_t* __restrict__ indices, int64_t* __restrict__ unique,
    int64_t* __restrict__ num_unique, const float* __restrict__ table, int64_t rows, int64_t dim,
    int g, float* __restrict__ out, int* __restrict__ status) {
  __shared__ int32_t pre[GPRE ? 1 : kFrLdsBlocks];
  __shared__ int32_t wsum[kFrWaves];
  __shared__ int64_t lkey[kFrThreads];
  __shared__ int32_t lnum[kFrThreads];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t i = (int64_t)blockIdx.x * kFrThreads + t;
  const int64_t ic = i < n ? i : n - 1;
  const int32_t f = fpos[ic];
  const int64_t key = keys[ic * stride];
  const int32_t fb = f >> kFrShift;
  int32_t p;  // exclusive prefix of f's block
  if constexpr (GPRE) {
    p = gpre[fb];
  } else {
    // prefix of the counts of blocks 0 .. (last position of the workgroup's block)
    const int64_t last = min((int64_t)(blockIdx.x + 1) * kFrThreads, n) - 1;
    const int64_t nb = (last >> kFrShift) + 1;
    int32_t carry = 0;
    for (int64_t base = 0; base < nb; base += kFrThreads) {
      const int64_t j = base + t;
      const int32_t v = j < nb ? count[j] : 0;
      int32_t total;
      const int32_t incl = fr_block_scan(v, wsum, &total);
      if (j < nb) pre[j] = carry + incl - v;
      carry += total;
    }
    __syncthreads();
    p = pre[fb];
    if (i == n - 1) num_unique[0] = carry;
  }
  const bool valid = i < n;
  const bool first = valid && f == static_cast<int32_t>(i);
  const int32_t r = p + rank[f] - 1;
  if (valid) indices[i] = r;
  if (first) unique[r] = key;
  if constexpr (GPRE) {
    if (i == n - 1) {  // the last block's prefix and count: the total
      const int64_t lb = (n - 1) >> kFrShift;
      num_unique[0] = gpre[lb] + count[lb];
    }
  }
  if (dim == 0) return;
  // list the workgroup's first occurrences in LDS, then copy their rows
  const uint64_t m = __ballot(first);
  const int rk = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                           __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
  if (lane == 0) wsum[w] = __popcll(m);
  __syncthreads();
  int before = 0, cnt = 0;
#pragma unroll
  for (int q = 0; q < kFrWaves; ++q) {
    before += q < w ? wsum[q] : 0;
    cnt += wsum[q];
  }
  if (first) {
    lkey[before + rk] = key;
    lnum[before + rk] = r;
  }
  __syncthreads();
  const int lane_g = t & (g - 1);
  for (int e = t / g; e < cnt; e += kFrThreads / g) {
    const int64_t id = lkey[e];
    const bool ok = id >= 0 && id < rows;
    if (!ok && lane_g == 0) atomicOr(status, 1);
    const float* src = table + (ok ? id : 0) * dim;
    float* dst = out + (int64_t)lnum[e] * dim;
    for (int64_t c = (int64_t)lane_g * VEC; c < dim; c += (int64_t)g * VEC) {
      if constexpr (VEC == 4) {
        typedef float V __attribute__((ext_vector_type(4)));
        const V v = ok ? *reinterpret_cast<const V*>(src + c) : V(0.0f);
        *reinterpret_cast<V*>(dst + c) = v;
      } else {
        dst[c] = ok ? src[c] : 0.0f;
      }
    }
  }
}

__global__ void store_i64_kernel(int64_t* p, int64_t v) { *p = v; }

// Workspace of the numbering: rank (n) and count (+ prefix beyond the LDS
// limit) as int32, each 256-byte aligned.
size_t fr_workspace(int64_t n) {
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const int64_t nblk = ceil_div(n, kFrBlock);
  return align(sizeof(int32_t) * (size_t)n) +
         align(sizeof(int32_t) * (size_t)nblk) * (nblk > kFrLdsBlocks ? 2 : 1);
}

// Numbers first occurrences given f (fpos receives f(i); it may be the
// array f reads), writes indices, unique, num_unique, and the rows of the
// unique keys when dim > 0.
template <class F>
int first_numbering(hipStream_t s, F first_of, const int64_t* keys, int64_t stride, int64_t n,
                    int32_t* fpos, char* ws, int64_t* num_unique, int64_t* unique,
                    int32_t* indices, const float* table, int64_t rows, int64_t dim, float* out,
                    int* status) {
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const int64_t nblk = ceil_div(n, kFrBlock);
  int32_t* rank = reinterpret_cast<int32_t*>(ws);
  int32_t* count = reinterpret_cast<int32_t*>(ws + align(sizeof(int32_t) * (size_t)n));
  int32_t* gpre = count + align(sizeof(int32_t) * (size_t)nblk) / sizeof(int32_t);
  const bool gp = nblk > kFrLdsBlocks;
  hipLaunchKernelGGL(fr_rank_kernel<F>, dim3((unsigned)nblk), dim3(kFrThreads), 0, s, first_of, n,
                     fpos, rank, count);
  ANNC_HIP_TRY(hipGetLastError());
  if (gp) {
    hipLaunchKernelGGL(fr_prefix_kernel, dim3(1), dim3(kFrThreads), 0, s, count, nblk, gpre);
    ANNC_HIP_TRY(hipGetLastError());
  }
  int g = 1;
  const bool vec = dim > 0 && dim % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const int64_t lanes = vec ? dim / 4 : dim;
  while (g < 64 && g < lanes) g <<= 1;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)ceil_div(n, kFrThreads)), dim3(kFrThreads), 0, s,
                       keys, stride, n, fpos,
                       rank, count, gpre, indices, unique, num_unique, table, rows, dim, g, out,
                       status);
  };
  if (vec)
    gp ? launch(fr_number_kernel<4, true>) : launch(fr_number_kernel<4, false>);
  else
    gp ? launch(fr_number_kernel<1, true>) : launch(fr_number_kernel<1, false>);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
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
  // eight independent loads in flight per step (a plain loop waited for
  // each load before issuing the next)
  int32_t m[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) m[j] = INT_MAX;
  int b = 0;
  for (; b + 8 <= nblk; b += 8) {
    int32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = part[(int64_t)(b + j) * range + r];
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = min(m[j], v[j]);
  }
  for (; b < nblk; ++b) m[0] = min(m[0], part[(int64_t)b * range + r]);
#pragma unroll
  for (int j = 1; j < 8; ++j) m[0] = min(m[0], m[j]);
  first[r] = m[0];
}

}  // namespace

int first_occurrence_range(hipStream_t s, const int64_t* keys, int64_t stride, int64_t n,
                           int64_t kmin, int64_t range, int64_t* num_unique, int64_t* unique,
                           int32_t* indices) {
  ANNC_REQUIRE(n > 0 && n < INT_MAX && range >= 1, "bad first-occurrence size");
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const int64_t nblk = ceil_div(n, kFoBlock);
  const bool local = range <= kFoLdsRange && nblk <= kFoMaxBlocks;
  const size_t fb = align(sizeof(int32_t) * (size_t)range);
  const size_t n4 = align(sizeof(int32_t) * (size_t)n);
  const size_t pb = local ? align(sizeof(int32_t) * (size_t)(nblk * range)) : 0;
  char* ws = static_cast<char*>(stream_workspace(s, fb + n4 + pb + fr_workspace(n)));
  if (!ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  int32_t* first = reinterpret_cast<int32_t*>(ws);
  int32_t* fpos = reinterpret_cast<int32_t*>(ws + fb);
  int32_t* part = reinterpret_cast<int32_t*>(ws + fb + n4);
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
  return first_numbering(s, FirstByKey{keys, stride, kmin, first}, keys, stride, n, fpos,
                         ws + fb + n4 + pb, num_unique, unique, indices, nullptr, 0, 0, nullptr,
                         status);
}

int unique_gather(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                  const int64_t* keys, int64_t stride, int64_t n, int64_t* num_unique,
                  int64_t* unique, int32_t* indices, float* out) {
  // Slot numbers, the empty marker `cap` included, are int32: cap <= 2^30.
  ANNC_REQUIRE(n <= kMaxUniqueKeys, "too many keys for the unique table (at most 2^29)");
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  int64_t cap = 1024;
  while (cap < 2 * n) cap <<= 1;
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t kb = align(sizeof(int64_t) * (size_t)(cap + 1));
  const size_t fb = align(sizeof(int32_t) * (size_t)(cap + 1));
  const size_t n4 = align(sizeof(int32_t) * (size_t)n);
  char* ws = static_cast<char*>(stream_workspace(s, kb + fb + n4 + fr_workspace(n)));
  if (!ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  int64_t* tab_key = reinterpret_cast<int64_t*>(ws);
  int32_t* tab_first = reinterpret_cast<int32_t*>(ws + kb);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws + kb + fb);
  hipLaunchKernelGGL(ug_clear_kernel, dim3((unsigned)ceil_div(cap + 1, kThreads)), dim3(kThreads),
                     0, s, tab_key, tab_first, cap + 1);
  ANNC_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(ug_insert_kernel, dim3((unsigned)ceil_div(n, kUgBlock)), dim3(kUgThreads), 0, s,
                     keys, stride, n, cap, tab_key, tab_first, slot_of, status);
  ANNC_HIP_TRY(hipGetLastError());
  // f(i) = tab_first[slot_of[i]], written over slot_of
  return first_numbering(s, FirstBySlot{slot_of, tab_first}, keys, stride, n, slot_of,
                         ws + kb + fb + n4, num_unique, unique, indices, table, rows, dim, out,
                         status);
}

}  // namespace annc

extern "C" int annc_hip_unique_gather(void* stream, const float* table, int64_t rows, int64_t dim,
                                      const int64_t* keys, int64_t key_stride, int64_t n,
                                      int64_t* num_unique, int64_t* unique, int32_t* indices,
                                      float* out) {
  using namespace annc;
  ANNC_REQUIRE(rows >= 0 && dim >= 0 && n >= 0 && key_stride >= 1, "bad dimensions");
  ANNC_REQUIRE(n <= kMaxUniqueKeys, "too many keys for the unique table (at most 2^29)");
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
