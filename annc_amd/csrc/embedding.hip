// embedding.hip -- embedding bags, segment reduction, masked gather and
// padded pooling on gfx950.
//
// Reference semantics (all CPU loops in ANNC):
//   * KPFusedSparseSegmentReduce
//     (annc/tensorflow/kernels/embedding_fused_sparse_segment_reduce.cc:87-151):
//     out[seg] accumulates data[idx] row by row in index order, per dim,
//     starting from 0.0f; mean multiplies by 1.0f/count.
//   * sparse_embedding2 kLoop fusion (annc/service/cpu/graph_opt.cc:8-41).
//   * __pooling (annc/service/cpu/graph_opt.cc:131-176).
//
// Bag kernel layout: a bag is owned by a group of G lanes of one wave64
// (G = dim/4 rounded up to a power of two, 4..64), each lane holding 4
// consecutive floats of the row, so a row is one contiguous G*16-byte
// (up to 1 KiB) read and one wave covers 64/G bags.  Every lane adds its
// rows in index order, which reproduces the reference's summation order
// exactly: the sum is bit-identical.  The ids and rows of up to kGroupRound
// positions are loaded before the first add, so they are in flight together.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "common.h"
#include "scan_sort.h"
#include "embedding_impl.h"

namespace annc {
namespace {

constexpr int kThreads = 256;
constexpr int kGroupRound = 32;  // bag positions whose loads are in flight together
constexpr int kQuarter = 8;  // granularity at which a round's row loads are skipped
constexpr uint32_t kNoRow = 0xffffffffu;  // row number of a masked bag position

// What masked bag positions read: zeros, so they add nothing.
// (a plain __device__ array, so that it shares the global address space
// with the table and selecting between the two keeps global loads).
__device__ __align__(16) float g_zero_vec[4] = {0.0f, 0.0f, 0.0f, 0.0f};

template <int VEC>
struct VecT;
template <>
struct VecT<4> {
  typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct VecT<2> {
  typedef float type __attribute__((ext_vector_type(2)));
};
template <>
struct VecT<1> {
  typedef float type;
};

template <int VEC>
__device__ __forceinline__ typename VecT<VEC>::type load_row(const float* p) {
  return *reinterpret_cast<const typename VecT<VEC>::type*>(p);
}

template <int VEC>
// Output rows are written once and read only by later kernels: non-temporal
// stores send them to memory without filling this XCD's L2, so the
// end-of-kernel release has no dirty output lines to write back.
__device__ __forceinline__ void store_row(float* p, typename VecT<VEC>::type v) {
  __builtin_nontemporal_store(v, reinterpret_cast<typename VecT<VEC>::type*>(p));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Raw buffer load of VEC floats at byte offset `off` of `rsrc`; offsets at or
// past the descriptor's byte count read zeros (hardware range check).
template <int VEC>
__device__ __forceinline__ typename VecT<VEC>::type buffer_row(__amdgpu_buffer_rsrc_t rsrc,
                                                               uint32_t off) {
  typedef typename VecT<VEC>::type V;
  if constexpr (VEC == 4) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(off), 0, 0);
    return __builtin_bit_cast(V, v);
  } else if constexpr (VEC == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rsrc, static_cast<int>(off), 0, 0);
    return __builtin_bit_cast(V, v);
  } else {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, static_cast<int>(off), 0, 0));
  }
}

// dword3 of a raw (untyped, stride 0) buffer descriptor on gfx950.
constexpr int kRawBufferFlags = 0x00020000;
// Byte offset that a masked bag position carries: the buffer path is used
// only for tables below 2 GiB, so it is always past the range check.
constexpr uint32_t kMaskedOff = 0x80000000u;

template <typename F, int... U>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, U...>) {
  (f(std::integral_constant<int, U>{}), ...);
}

// The value `v` holds in lane U of this lane's aligned group of G lanes.
// For G = 16 the group is a DPP row and row_newbcast is one VALU move;
// other widths go through the LDS permute network (ds_bpermute).
template <int G, int U>
__device__ __forceinline__ uint32_t group_bcast(uint32_t v) {
  if constexpr (G == 16)
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x150 + U, 0xF, 0xF, false));
  else
    return static_cast<uint32_t>(__shfl(static_cast<int>(v), U, G));
}


// x moved by the DPP control CTRL into the rows of ROW_MASK (lanes with no
// source lane, and rows outside the mask, read 0).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_move(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, 0xf, false));
}

// Inclusive sum over the lanes of a wave64 by DPP moves: rows of 16 by
// row_shr 1, 2, 4 and 8, then lane 15's row total into rows 1 and 3
// (row_bcast:15) and lane 31's into rows 2 and 3 (row_bcast:31).  Six VALU
// moves instead of six LDS permutes; every add is unconditional, as a lane
// with no source reads 0.
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
  v += dpp_move<0x111, 0xf>(v);
  v += dpp_move<0x112, 0xf>(v);
  v += dpp_move<0x114, 0xf>(v);
  v += dpp_move<0x118, 0xf>(v);
  v += dpp_move<0x142, 0xa>(v);
  v += dpp_move<0x143, 0xc>(v);
  return v;
}

// The value of lane 63 (scalar read).
__device__ __forceinline__ uint32_t lane63(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Row ids of bag positions from global memory: ids[at] or, through a
// permutation, ids[perm[at]] (every slot loaded: the clamped positions are
// valid; permuted positions first, then the ids they name, so each level is
// waited for once).
template <typename IdxT, bool PERM>
struct GlobalIds {
  const IdxT* ids;
  const int32_t* perm;
  template <int K>
  __device__ __forceinline__ void operator()(int64_t (&at)[K], const bool (&loaded)[K],
                                             int64_t (&idv)[K]) const {
    if constexpr (PERM) {
#pragma unroll
      for (int t = 0; t < K; ++t) at[t] = perm[at[t]];
#pragma unroll
      for (int t = 0; t < K; ++t) idv[t] = static_cast<int64_t>(ids[at[t]]);
    } else {
#pragma unroll
      for (int t = 0; t < K; ++t) idv[t] = loaded[t] ? static_cast<int64_t>(ids[at[t]]) : 0;
    }
  }
};

// Row ids of bag positions from an LDS copy of ids[w0, w0 + wn) when every
// position the wave asks for lies there, else from global memory (the
// choice is made per wave, so either way the loads need no per-lane branch).
template <typename IdxT>
struct WindowIds {
  const IdxT* ids;
  const IdxT* win;  // LDS
  int64_t w0, wn;
  template <int K>
  __device__ __forceinline__ void operator()(int64_t (&at)[K], const bool (&loaded)[K],
                                             int64_t (&idv)[K]) const {
    bool out = false;
#pragma unroll
    for (int t = 0; t < K; ++t)
      out |= loaded[t] && static_cast<uint64_t>(at[t] - w0) >= static_cast<uint64_t>(wn);
    if (__ballot(out) == 0) {
#pragma unroll
      for (int t = 0; t < K; ++t) idv[t] = loaded[t] ? static_cast<int64_t>(win[at[t] - w0]) : 0;
    } else {
#pragma unroll
      for (int t = 0; t < K; ++t) idv[t] = loaded[t] ? static_cast<int64_t>(ids[at[t]]) : 0;
    }
  }
};

// One bag, reduced by this lane's aligned group of G lanes (every lane of
// the group calls it with the same bag; groups of a wave may hold different
// bags).  The bag is walked in rounds of kGroupRound positions: the round's
// ids are fetched (clamped into the bag, so every load is valid and no
// per-position exec mask is needed; lanes fetch distinct ids and broadcast
// them inside the group), then all of the round's row chunks, and only then
// are the first `cnt` rows added in index order.  A bag of n ids costs
// ceil(n/32) id->row round trips.  Returns true if an id was outside the
// table.
template <int G, int VEC, bool MEAN, bool BUF, typename Fetch>
__device__ __forceinline__ bool bag_group(const float* __restrict__ table, int64_t rows,
                                          int64_t dim, int64_t beg, int64_t end,
                                          const Fetch& fetch, float* __restrict__ out_row) {
  typedef typename VecT<VEC>::type V;
  const int g = threadIdx.x & (G - 1);
  bool bad = false;
  // Every lane of the group runs the same chunk and round loops (the row
  // broadcasts read all G lanes); lanes past `dim` read the zero vector.
  const uint32_t row_bytes = static_cast<uint32_t>(dim * sizeof(float));
  // BUF: the table is below 2 GiB, reached through a raw buffer descriptor
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(table), 0, static_cast<int>(BUF ? rows * row_bytes : 0), kRawBufferFlags);
  for (int64_t c0 = 0; c0 < dim; c0 += (int64_t)G * VEC) {
    const int64_t c = c0 + (int64_t)g * VEC;
    const bool active = c < dim;
    const char* base = reinterpret_cast<const char*>(table + (active ? c : 0));
    const char* zero = reinterpret_cast<const char*>(g_zero_vec);
    // buffer path: byte offset of this lane's chunk; inactive lanes push every
    // offset past the range check
    const uint32_t c_off = active ? static_cast<uint32_t>(c * sizeof(float)) : kMaskedOff;
    V acc = V(0.0f);
    for (int64_t j0 = beg; j0 < end; j0 += kGroupRound) {
      const int cnt = static_cast<int>(end - j0 < kGroupRound ? end - j0 : kGroupRound);
      // Only the parts of the round that some bag of this wave reaches are
      // loaded: id slot t if a bag has more than G*t positions left, row
      // quarter q (positions 8q..8q+7) if one has more than 8q.
      constexpr int kPer = (kGroupRound + G - 1) / G;
      constexpr int kQuarters = kGroupRound / kQuarter;
      constexpr uint32_t kMasked = BUF ? kMaskedOff : kNoRow;
      // Lane g of the group fetches positions g, g+G, ... of the round (one
      // coalesced load per slot) and turns each into a byte offset (BUF) or a
      // 32-bit row number, or the masked value for positions past the bag,
      // ids outside the table and slots no bag of the wave reaches.
      // (all of the round's id loads are issued before any is used, so the
      // conversion below waits for them once)
      int64_t idv[kPer];
      bool loaded[kPer];
      int64_t at[kPer];
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        loaded[t] = t == 0 || __ballot(cnt > G * t) != 0;
        at[t] = j0 + min(g + G * t, cnt - 1);
      }
      fetch(at, loaded, idv);
      uint32_t mine[kPer];
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const bool in_bag = loaded[t] && g + G * t < cnt;
        const bool ok = static_cast<uint64_t>(idv[t]) < static_cast<uint64_t>(rows);
        bad |= in_bag && !ok;
        const uint32_t row = static_cast<uint32_t>(idv[t]);
        mine[t] = (in_bag && ok) ? (BUF ? row * row_bytes : row) : kMasked;
      }
      // position u comes from lane u % G, slot u / G; masked positions read
      // zeros, so the adds need no mask (x + 0.0f == x for the +0-seeded sums)
      V v[kGroupRound];
      bool need[kQuarters];
      static_for([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        need[q] = q == 0 || __ballot(cnt > kQuarter * q) != 0;
        if (need[q]) {
          static_for([&](auto uc) {
            constexpr int u = kQuarter * q + decltype(uc)::value;
            if constexpr (BUF) {
              v[u] = buffer_row<VEC>(rsrc, group_bcast<G, u % G>(mine[u / G]) + c_off);
            } else {
              const uint32_t row = group_bcast<G, u % G>(mine[u / G]);
              const bool take = row != kNoRow && active;
              const uint64_t off = static_cast<uint64_t>(take ? row : 0u) * row_bytes;
              const char* src = (take ? base : zero) + off;
              v[u] = load_row<VEC>(reinterpret_cast<const float*>(src));
            }
          }, std::make_integer_sequence<int, kQuarter>{});
        }
      }, std::make_integer_sequence<int, kQuarters>{});
      static_for([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        if (need[q]) {
#pragma unroll
          for (int u = kQuarter * q; u < kQuarter * (q + 1); ++u) acc += v[u];
        }
      }, std::make_integer_sequence<int, kQuarters>{});
    }
    if (MEAN) {
      const int32_t n = static_cast<int32_t>(end - beg);
      if (n > 0) acc *= 1.0f / static_cast<float>(n);
    }
    if (active) store_row<VEC>(out_row + c, acc);
  }
  return bad;
}

// Threads of a bag-kernel workgroup (configs[2], sum: 128 and 256 threads
// measure alike, 3.33 and 3.35 us; 512 takes 4.09 us).
constexpr int kBagThreads = 256;

// One bag per group of G lanes (64/G bags share a wave).
template <typename IdxT, int G, int VEC, bool MEAN, bool PERM, bool BUF>
__global__ __launch_bounds__(kBagThreads) void bag_kernel(
    const float* __restrict__ table, int64_t rows, int64_t dim, const IdxT* __restrict__ ids,
    const int32_t* __restrict__ perm, const int64_t* __restrict__ offsets, int64_t num_bags,
    float* __restrict__ out, int64_t ldo, int* __restrict__ status) {
  const int64_t bag = ((int64_t)blockIdx.x * kBagThreads + threadIdx.x) / G;
  if (bag >= num_bags) return;
  const bool bad = bag_group<G, VEC, MEAN, BUF>(table, rows, dim, offsets[bag], offsets[bag + 1],
                                                GlobalIds<IdxT, PERM>{ids, perm}, out + bag * ldo);
  if (bad) atomicOr(status, 1);
}

template <typename IdxT, int G, int VEC>
int launch_bag_g(const BagArgs& a, hipStream_t s) {
  const int64_t threads = a.num_bags * G;
  dim3 grid((unsigned)ceil_div(threads, kBagThreads));
  const IdxT* ids = static_cast<const IdxT*>(a.ids);
  const bool mean = a.combiner == ANNC_COMBINER_MEAN;
  // tables below 2 GiB go through the buffer path (masked positions read the
  // range check's zeros)
  const bool buf = a.rows * a.dim * static_cast<int64_t>(sizeof(float)) < (int64_t(1) << 31);
  auto pick = [&](auto buf_tag) {
    constexpr bool B = decltype(buf_tag)::value;
    return a.perm ? (mean ? bag_kernel<IdxT, G, VEC, true, true, B> : bag_kernel<IdxT, G, VEC, false, true, B>)
                  : (mean ? bag_kernel<IdxT, G, VEC, true, false, B> : bag_kernel<IdxT, G, VEC, false, false, B>);
  };
  auto kernel = buf ? pick(std::true_type{}) : pick(std::false_type{});
  hipLaunchKernelGGL(kernel, grid, dim3(kBagThreads), 0, s, a.table, a.rows, a.dim, ids, a.perm,
                     a.offsets, a.num_bags, a.out, a.ldo, a.status);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

template <typename IdxT, int VEC>
int launch_bag_vec(const BagArgs& a, hipStream_t s) {
  const int64_t lanes = ceil_div(a.dim, VEC);
  if (lanes <= 4) return launch_bag_g<IdxT, 4, VEC>(a, s);
  if (lanes <= 8) return launch_bag_g<IdxT, 8, VEC>(a, s);
  if (lanes <= 16) return launch_bag_g<IdxT, 16, VEC>(a, s);
  if (lanes <= 32) return launch_bag_g<IdxT, 32, VEC>(a, s);
  return launch_bag_g<IdxT, 64, VEC>(a, s);
}

template <typename IdxT>
int launch_bag_idx(const BagArgs& a, hipStream_t s) {
  auto aligned = [](const void* p, int bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
  };
  auto vec_ok = [&](int v) {
    return a.dim % v == 0 && a.ldo % v == 0 && aligned(a.table, 4 * v) && aligned(a.out, 4 * v);
  };
  return vec_ok(4) ? launch_bag_vec<IdxT, 4>(a, s) : launch_bag_vec<IdxT, 1>(a, s);
}

// ---------------------------------------------------------------------------
// Segment reduction over non-decreasing segment ids in one launch, without
// an offsets pass.  Ids are clamped to [-1, batch] (positions outside
// [0, batch) belong to no segment) and position n is a closing sentinel of
// id `batch`.  A position whose id differs from the one before it is a
// boundary: the segments strictly between the two ids hold no positions and
// get zero rows, and if its id is a segment, that segment starts there and
// runs to the next boundary.  Workgroup w owns the boundaries at positions
// [w*P, (w+1)*P): it lists them in LDS in position order, finds where its
// last segment ends by reading ahead P positions past its chunk, and hands
// its segments to its groups of G lanes, which reduce them in index order as
// the bag kernel does.  The row ids of those 2P positions are read in the
// same round as their segment ids and kept in LDS, so a segment that ends
// inside them waits for one global round (its rows) after the boundaries:
// two dependent rounds in all, against the offsets kernel plus the bag
// kernel's three (offsets, row ids, rows).
// ---------------------------------------------------------------------------
// Positions per workgroup (at most kThreads): 160 keeps a chunk's segments
// (20 positions each in configs[2]) within the 16 lane groups of a
// workgroup, so none takes a second turn (256 gives the chunks with more
// than 16 segments a second turn).  configs[2], us per launch: 64 positions
// 5.25, 96 5.38, 128 4.64, 160 4.45, 192 4.65.
constexpr int kSsChunk = 160;

template <typename IdxT, int G, int VEC, bool MEAN, bool BUF, int P = kSsChunk>
__global__ __launch_bounds__(kThreads) void seg_sorted_kernel(
    const float* __restrict__ table, int64_t rows, int64_t dim, const IdxT* __restrict__ ids,
    const int64_t* __restrict__ seg, int64_t stride, int64_t n, int64_t batch,
    float* __restrict__ out, int64_t ldo, int* __restrict__ status) {
  typedef typename VecT<VEC>::type V;
  constexpr int kWaves = kThreads / 64;
  static_assert(P <= kThreads, "one position per thread");
  __shared__ int32_t bpos[P];
  __shared__ int64_t bkey[P];
  __shared__ int64_t bprev[P];
  __shared__ int32_t wcnt[kWaves];
  __shared__ int32_t wend[kWaves];
  __shared__ int32_t wgap[kWaves];
  __shared__ IdxT win[2 * P];  // row ids of positions [p0, p0 + 2P)
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t p0 = (int64_t)blockIdx.x * P;
  const int64_t p1 = p0 + P;
  // Ids are loaded from a clamped, always valid position and fixed up once
  // all loads are issued, so no load sits in a per-lane branch.
  auto load = [&](int64_t j) -> int64_t {
    return seg[(j < 0 ? 0 : (j >= n ? n - 1 : j)) * stride];
  };
  auto fix = [&](int64_t j, int64_t v) -> int64_t {
    return j < 0 ? int64_t(-1)
                 : (j >= n ? batch : (v < -1 ? int64_t(-1) : (v > batch ? batch : v)));
  };
  auto key = [&](int64_t j) { return fix(j, load(j)); };
  // this position and the one before it, and the same a chunk ahead (no
  // positions at all: every id is the sentinel's)
  const int64_t i = p0 + t;
  int64_t prev = batch, cur = batch, ahead_prev = batch, ahead = batch;
  if (n > 0) {
    // the row ids of the chunk and of the read-ahead come in the same round,
    // into LDS: the segments then wait for their rows only
    const IdxT d0 = ids[i < n ? i : n - 1], d1 = ids[p1 + t < n ? p1 + t : n - 1];
    const int64_t v0 = load(i - 1), v1 = load(i), v2 = load(p1 + t - 1), v3 = load(p1 + t);
    if (t < P) {
      win[t] = d0;
      win[P + t] = d1;
    }
    prev = fix(i - 1, v0);
    cur = fix(i, v1);
    ahead_prev = fix(p1 + t - 1, v2);
    ahead = fix(p1 + t, v3);
  }
  if (i == 0) prev = -1;
  const bool bnd = t < P && i <= n && cur != prev;
  const uint64_t m = __ballot(bnd);
  const int rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
  const uint64_t ma = __ballot(t < P && ahead != ahead_prev);
  const uint64_t mg = __ballot(bnd && cur > prev + 1);
  if (lane == 0) {
    wcnt[w] = __popcll(m);
    // (a segment's end is at most n: candidates are clamped there, so the
    // int never wraps)
    wend[w] = ma ? (int)min(p1 + 64 * w + __builtin_ctzll(ma), n) : INT32_MAX;
    wgap[w] = mg != 0;
  }
  __syncthreads();
  int before = 0, nb = 0, any_gap = 0;
  int32_t end_last = INT32_MAX;
#pragma unroll
  for (int q = 0; q < kWaves; ++q) {
    before += q < w ? wcnt[q] : 0;
    nb += wcnt[q];
    any_gap |= wgap[q];
    end_last = wend[q] < end_last ? wend[q] : end_last;
  }
  if (bnd) {
    bpos[before + rank] = static_cast<int32_t>(i);
    bkey[before + rank] = cur;
    bprev[before + rank] = prev;
  }
  __syncthreads();
  if (nb == 0) return;
  // The last listed segment, when it is one, ends at the first boundary past
  // the chunk: found above unless it lies beyond the read-ahead (a segment
  // longer than the chunk), then searched for a chunk at a time.  It exists:
  // position n closes every segment.
  const int64_t last = bkey[nb - 1];
  if (last >= 0 && last < batch) {
    for (int64_t base = p1 + P; end_last == INT32_MAX; base += kThreads) {
      const uint64_t mb = __ballot(key(base + t) != last);
      __syncthreads();
      if (lane == 0) wend[w] = mb ? (int)min(base + 64 * w + __builtin_ctzll(mb), n) : INT32_MAX;
      __syncthreads();
#pragma unroll
      for (int q = 0; q < kWaves; ++q) end_last = wend[q] < end_last ? wend[q] : end_last;
    }
  }
  // zero rows for the segments that no position names
  if (any_gap) {
    const int64_t dv = dim / VEC;
    for (int k = 0; k < nb; ++k) {
      const int64_t lo = bprev[k] + 1, hi = bkey[k] < batch ? bkey[k] : batch;
      for (int64_t e = t; e < (hi - lo) * dv; e += kThreads) {
        const int64_t r = lo + e / dv;
        store_row<VEC>(out + r * ldo + (e % dv) * VEC, V(0.0f));
      }
    }
  }
  bool bad = false;
  const int64_t wn = n - p0 < 2 * P ? n - p0 : 2 * P;
  for (int k = t / G; k < nb; k += kThreads / G) {
    const int64_t sk = bkey[k];
    if (sk < 0 || sk >= batch) continue;
    const int64_t beg = bpos[k], end = k + 1 < nb ? bpos[k + 1] : end_last;
    bad |= bag_group<G, VEC, MEAN, BUF>(table, rows, dim, beg, end,
                                        WindowIds<IdxT>{ids, win, p0, wn}, out + sk * ldo);
  }
  if (bad) atomicOr(status, 1);
}

template <typename IdxT, int G, int VEC>
int launch_seg_sorted_g(const BagArgs& a, const int64_t* seg, int64_t stride, int64_t n,
                        hipStream_t s) {
  const IdxT* ids = static_cast<const IdxT*>(a.ids);
  const bool mean = a.combiner == ANNC_COMBINER_MEAN;
  const bool buf = a.rows * a.dim * static_cast<int64_t>(sizeof(float)) < (int64_t(1) << 31);
  auto pick = [&](auto buf_tag) {
    constexpr bool B = decltype(buf_tag)::value;
    return mean ? seg_sorted_kernel<IdxT, G, VEC, true, B> : seg_sorted_kernel<IdxT, G, VEC, false, B>;
  };
  auto kernel = buf ? pick(std::true_type{}) : pick(std::false_type{});
  // one workgroup per kSsChunk positions, position n (the sentinel) included
  const dim3 grid((unsigned)(n / kSsChunk + 1));
  hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, a.table, a.rows, a.dim, ids, seg, stride,
                     n, a.num_bags, a.out, a.ldo, a.status);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

template <typename IdxT, int VEC>
int launch_seg_sorted_vec(const BagArgs& a, const int64_t* seg, int64_t stride, int64_t n,
                          hipStream_t s) {
  const int64_t lanes = ceil_div(a.dim, VEC);
  if (lanes <= 4) return launch_seg_sorted_g<IdxT, 4, VEC>(a, seg, stride, n, s);
  if (lanes <= 8) return launch_seg_sorted_g<IdxT, 8, VEC>(a, seg, stride, n, s);
  if (lanes <= 16) return launch_seg_sorted_g<IdxT, 16, VEC>(a, seg, stride, n, s);
  if (lanes <= 32) return launch_seg_sorted_g<IdxT, 32, VEC>(a, seg, stride, n, s);
  return launch_seg_sorted_g<IdxT, 64, VEC>(a, seg, stride, n, s);
}

template <typename IdxT>
int launch_seg_sorted(const BagArgs& a, const int64_t* seg, int64_t stride, int64_t n,
                      hipStream_t s) {
  auto aligned = [](const void* p, int bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
  };
  const bool v4 = a.dim % 4 == 0 && a.ldo % 4 == 0 && aligned(a.table, 16) && aligned(a.out, 16);
  return v4 ? launch_seg_sorted_vec<IdxT, 4>(a, seg, stride, n, s)
            : launch_seg_sorted_vec<IdxT, 1>(a, seg, stride, n, s);
}

// ---------------------------------------------------------------------------
// Segment-id preprocessing for unsorted segment reduction.
// ---------------------------------------------------------------------------
// Partial min, max and "some id is smaller than the one before it" of
// seg[i*stride] over each block's grid-stride share, one record per block
// (no atomics: the host combines the blocks' records).
__global__ __launch_bounds__(kThreads) void seg_scan_kernel(const int64_t* __restrict__ seg,
                                                           int64_t stride, int64_t n,
                                                           long long* __restrict__ part) {
  __shared__ long long red[3][kThreads / 64];
  long long lo = LLONG_MAX, hi = LLONG_MIN;
  int unsort = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const long long v = seg[i * stride];
    lo = v < lo ? v : lo;
    hi = v > hi ? v : hi;
    if (i > 0 && v < seg[(i - 1) * stride]) unsort = 1;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const long long l2 = __shfl_xor(lo, off, 64);
    const long long h2 = __shfl_xor(hi, off, 64);
    lo = l2 < lo ? l2 : lo;
    hi = h2 > hi ? h2 : hi;
    unsort |= __shfl_xor(unsort, off, 64);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = lo;
    red[1][w] = hi;
    red[2][w] = unsort;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < kThreads / 64; ++q) {
      lo = red[0][q] < lo ? red[0][q] : lo;
      hi = red[1][q] > hi ? red[1][q] : hi;
      unsort |= static_cast<int>(red[2][q]);
    }
    part[3 * blockIdx.x] = lo;
    part[3 * blockIdx.x + 1] = hi;
    part[3 * blockIdx.x + 2] = unsort;
  }
}

// offsets[s] = first position whose segment id is >= s, for s in [0, batch],
// from non-decreasing segment ids: position i fills the s in
// (seg[i-1], seg[i]] (ids clamped to [-1, batch]; i = n closes the range).
template <typename KeyT>
__global__ void seg_bounds_kernel(const KeyT* __restrict__ seg, int64_t stride, int64_t n,
                                  int64_t batch, int64_t* __restrict__ offsets) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i > n) return;
  auto key = [&](int64_t j) {
    const int64_t v = static_cast<int64_t>(seg[j * stride]);
    return v < -1 ? int64_t(-1) : (v > batch ? batch : v);
  };
  const int64_t prev = i == 0 ? int64_t(-1) : key(i - 1);
  const int64_t cur = i == n ? batch : key(i);
  for (int64_t s = prev + 1; s <= cur; ++s) offsets[s] = i;
}

// ---------------------------------------------------------------------------
// Stable counting sort of positions by segment id, for segment ids below
// kCsMaxSegments (the per-block counters live in LDS).  Positions are cut
// into blocks of kCsBlock:
//   1. cs_hist:    H[b][s] = positions of block b in segment s
//   2. cs_prefix:  P[b][s] = positions of segment s in blocks before b,
//                  total[s]
//   3. cs_offsets: offsets = exclusive scan of total (one workgroup)
//   4. cs_scatter: one wave per block walks its positions in order, 64 at a
//                  time; lanes holding the same segment rank themselves by
//                  lane order (ballots over the id bits), so each segment's
//                  positions land in increasing order: perm is stable.
// Segment ids outside [0, batch) are left out, as the sort path leaves them
// past offsets[batch].
// ---------------------------------------------------------------------------
constexpr int kCsBlock = 1024;
constexpr int64_t kCsMaxSegments = 16384;
constexpr int kCsBits = 14;  // bits of a segment id below kCsMaxSegments

__global__ __launch_bounds__(kThreads) void cs_hist_kernel(const int64_t* __restrict__ seg,
                                                          int64_t stride, int64_t n, int batch,
                                                          uint32_t* __restrict__ H) {
  extern __shared__ uint32_t cs_lds[];
  for (int s = threadIdx.x; s < batch; s += kThreads) cs_lds[s] = 0;
  __syncthreads();
  const int64_t b0 = (int64_t)blockIdx.x * kCsBlock;
  // every id of the thread is loaded (positions clamped to n - 1) before the
  // first count, so the loads travel together
  constexpr int kPer = kCsBlock / kThreads;
  int64_t sv[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t i = b0 + threadIdx.x + u * kThreads;
    sv[u] = seg[(i < n ? i : n - 1) * stride];
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int64_t i = b0 + threadIdx.x + u * kThreads;
    if (i < n && sv[u] >= 0 && sv[u] < batch) atomicAdd(&cs_lds[sv[u]], 1u);
  }
  __syncthreads();
  uint32_t* row = H + (int64_t)blockIdx.x * batch;
  for (int s = threadIdx.x; s < batch; s += kThreads) row[s] = cs_lds[s];
}

// P[b][s] = sum of H[b'][s] over blocks b' < b, total[s] = the sum over all
// blocks.  A workgroup of 1024 threads takes 64 segments (one per lane, so
// every load is a 256-byte row segment) and splits the blocks into 16
// chunks, one per wave: each wave sums its chunk, the chunk sums meet in LDS,
// and each wave then writes its chunk's running prefixes from its own
// offset.  The counts are read once from HBM and once more from L2.
__global__ __launch_bounds__(1024) void cs_prefix_kernel(const uint32_t* __restrict__ H,
                                                       int batch, int nblk,
                                                       uint32_t* __restrict__ P,
                                                       uint32_t* __restrict__ total) {
  __shared__ uint32_t part[16][64];
  constexpr int U = 8;  // counts in flight per thread
  const int j = threadIdx.x & 63, c = threadIdx.x >> 6;
  const int s = blockIdx.x * 64 + j;
  const bool ok = s < batch;
  const int per = (nblk + 15) / 16;
  const int b_lo = min(nblk, c * per), b_hi = min(nblk, b_lo + per);
  // loads are unconditional (block and segment clamped into range) and
  // masked afterwards, so the U loads of a step travel together
  const int sc = ok ? s : batch - 1;
  uint32_t sum = 0;
  for (int b = b_lo; b < b_hi; b += U) {
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = H[(int64_t)min(b + u, b_hi - 1) * batch + sc];
#pragma unroll
    for (int u = 0; u < U; ++u) sum += (ok && b + u < b_hi) ? v[u] : 0u;
  }
  part[c][j] = sum;
  __syncthreads();
  uint32_t run = 0;
  for (int q = 0; q < c; ++q) run += part[q][j];
  if (ok && c == 15) total[s] = run + sum;
  if (!ok) return;
  for (int b = b_lo; b < b_hi; b += U) {
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = H[(int64_t)min(b + u, b_hi - 1) * batch + s];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (b + u < b_hi) P[(int64_t)(b + u) * batch + s] = run;
      run += b + u < b_hi ? v[u] : 0u;
    }
  }
}

// Exclusive scan of the segment totals (batch <= kCsMaxSegments = 16 * 1024,
// so each thread keeps its at most 16 totals in registers).
__global__ __launch_bounds__(1024) void cs_offsets_kernel(const uint32_t* __restrict__ total,
                                                         int batch, int64_t* __restrict__ offsets) {
  __shared__ int64_t wave_tot[16];
  constexpr int kMaxPer = 16;
  const int per = (batch + 1023) / 1024;
  const int s0 = threadIdx.x * per;
  uint32_t tv[kMaxPer];
#pragma unroll
  for (int u = 0; u < kMaxPer; ++u) tv[u] = (u < per && s0 + u < batch) ? total[s0 + u] : 0u;
  int64_t sum = 0;
#pragma unroll
  for (int u = 0; u < kMaxPer; ++u) sum += tv[u];
  // inclusive scan of the thread sums: within each wave by shuffles, then
  // over the 16 wave totals through LDS
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t incl = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int64_t before = 0;
  for (int q = 0; q < wave; ++q) before += wave_tot[q];
  int64_t run = before + incl - sum;  // exclusive prefix of this thread
#pragma unroll
  for (int u = 0; u < kMaxPer; ++u) {
    if (u < per && s0 + u < batch) offsets[s0 + u] = run;
    run += tv[u];
  }
  if (threadIdx.x == 1023) offsets[batch] = before + incl;
}

__global__ __launch_bounds__(kThreads) void cs_scatter_kernel(const int64_t* __restrict__ seg,
                                                             int64_t stride, int64_t n, int batch,
                                                             const uint32_t* __restrict__ P,
                                                             const int64_t* __restrict__ offsets,
                                                             int32_t* __restrict__ perm) {
  extern __shared__ uint32_t cs_lds[];  // next slot of each segment
  const uint32_t* pre = P + (int64_t)blockIdx.x * batch;
  // cursor loads in flight per thread; unconditional (segment clamped to
  // batch - 1), so they are issued together and waited for once
  constexpr int kInit = 16;
  for (int s0 = threadIdx.x; s0 < batch; s0 += kThreads * kInit) {
    uint32_t v[kInit];
#pragma unroll
    for (int u = 0; u < kInit; ++u) {
      const int s = min(s0 + u * kThreads, batch - 1);
      v[u] = static_cast<uint32_t>(offsets[s]) + pre[s];
    }
#pragma unroll
    for (int u = 0; u < kInit; ++u) {
      const int s = s0 + u * kThreads;
      if (s < batch) cs_lds[s] = v[u];
    }
  }
  __syncthreads();
  if (threadIdx.x >= 64) return;
  // One wave walks the block in order.  LDS operations of a wave complete
  // in program order, so each step sees the cursors the previous one left.
  const int lane = threadIdx.x;
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  const int64_t b0 = (int64_t)blockIdx.x * kCsBlock;
  // every segment id of the block is fetched before the ordered walk
  constexpr int T = kCsBlock / 64;
  int64_t sv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t i = b0 + 64 * t + lane;
    sv[t] = i < n ? seg[i * stride] : -1;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t i = b0 + 64 * t + lane;
    const int64_t s = sv[t];
    const bool ok = s >= 0 && s < batch;
    uint64_t same = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < kCsBits; ++bit) {
      const bool on = (s >> bit) & 1;
      const uint64_t b = __ballot(on);
      same &= on ? b : ~b;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(same & lt));
    const uint32_t cnt = static_cast<uint32_t>(__popcll(same));
    const uint32_t base = ok ? cs_lds[s] : 0u;
    if (ok) {
      perm[base + rank] = static_cast<int32_t>(i);
      if (rank + 1 == cnt) cs_lds[s] = base + cnt;
    }
  }
}

// ---------------------------------------------------------------------------
// Two-level stable sort of positions by segment (at most kCsMaxSegments
// segments and kTlMaxBlocks blocks of positions), in two launches before
// the bag kernel:
//   1. seg_block_sort: each block of kTlBlock positions is sorted by segment
//      range (bucket = segment / S; ids outside [0, batch) get the key
//      kTlBuckets and are left out), stably: equal buckets keep their
//      position order.  It writes the sorted positions, their segments, and
//      bstart[block][b], the first sorted index of bucket b (b < kTlBuckets;
//      bstart[block][kTlBuckets] counts the kept positions).
//   2. seg_range: workgroup g owns the S segments of bucket g and takes the
//      slice [bstart[a][g], bstart[a][g+1]) of every block a.  Blocks in
//      order, each slice in position order: the concatenation is in position
//      order.  The sum of bstart[a][g] over the blocks counts the kept
//      positions of the buckets before g, which is where the range starts in
//      perm, so no workgroup waits for another.  It ranks its positions by
//      segment in LDS (ballot match over log2(S) bits, 64 entries per wave
//      step, as cs_scatter) and writes perm and its segments' offsets.
// ---------------------------------------------------------------------------
constexpr int kTlThreads = 256;
constexpr int kTlWaves = kTlThreads / 64;
constexpr int kTlItems = 4;
constexpr int kTlBlock = kTlThreads * kTlItems;  // positions per block
constexpr int kTlBuckets = 256;                   // segment ranges
constexpr int kTlBucketBits = 9;                  // bucket kTlBuckets: dropped ids
constexpr int kTlMaxBlocks = 4096;                // up to 4 Mi positions
constexpr int kTlPer = kTlMaxBlocks / kTlThreads; // blocks per thread in step 2
constexpr int kTlCap = 8192;                      // step 2's list (LDS)
constexpr int kTlMaxS = 64;                       // segments per range
constexpr int kTlMaxSBits = 6;
static_assert(kCsMaxSegments <= int64_t(kTlBuckets) * kTlMaxS, "segment ranges");

// ROWS: the row id of every sorted position (indices[p], or 0xffffffff for
// an id outside [0, rows)) instead of the position, for the fused reduction
// of step 2.  THREADS x ITEMS positions per block, NB buckets (NB <= THREADS;
// KEYBITS bits hold the keys 0..NB, NB marking a dropped position);
// bstart[block][b] has NB + 1 entries per block.
template <typename IdxT, bool ROWS, int THREADS, int ITEMS, int NB, int KEYBITS>
__global__ __launch_bounds__(THREADS) void seg_block_sort_kernel(
    const int64_t* __restrict__ seg, int64_t stride, int64_t n, int batch, int S,
    const IdxT* __restrict__ indices, int64_t rows, uint32_t* __restrict__ sorted_pos,
    uint16_t* __restrict__ sorted_seg, uint32_t* __restrict__ sorted_row,
    uint32_t* __restrict__ bstart) {
  static_assert(NB <= THREADS && (1 << KEYBITS) > NB, "bucket keys");
  constexpr int kWaves = THREADS / 64;
  constexpr int kBlock = THREADS * ITEMS;
  // Positions are striped (item i of thread t is position b0 + i*THREADS + t),
  // so the wave steps (i, wave) taken in order visit positions in order.
  // Each step ranks its lanes per bucket by a ballot match over the key
  // bits; cnt[b][step] holds the step's bucket counts (a bucket's counts are
  // 32 contiguous bytes, read and written as two 16-byte words).  An entry's
  // slot is then start[b] + (b's entries in the steps before) + its rank.
  constexpr int kSteps = ITEMS * kWaves;
  static_assert(kSteps == 16, "a bucket's step counts are two 16-byte LDS words");
  __shared__ __align__(16) uint16_t cnt[NB + 1][kSteps];
  __shared__ uint32_t start[NB + 1];
  __shared__ uint32_t wsum[kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  const int64_t b0 = (int64_t)blockIdx.x * kBlock;
  // unconditional loads (position clamped to n - 1), so they travel together
  int64_t v[ITEMS], iv[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t p = b0 + i * THREADS + t;
    v[i] = seg[(p < n ? p : n - 1) * stride];
    if constexpr (ROWS) iv[i] = static_cast<int64_t>(indices[p < n ? p : n - 1]);
  }
  u32x4* cwords = reinterpret_cast<u32x4*>(&cnt[0][0]);
  for (int k = t; k < 2 * (NB + 1); k += THREADS) cwords[k] = u32x4(0u);
  uint32_t key[ITEMS], rank[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int64_t p = b0 + i * THREADS + t;
    const bool ok = p < n && v[i] >= 0 && v[i] < batch;
    key[i] = ok ? static_cast<uint32_t>(v[i]) / static_cast<uint32_t>(S) : NB;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    uint64_t same = ~uint64_t(0);
#pragma unroll
    for (int bit = 0; bit < KEYBITS; ++bit) {
      const bool on = (key[i] >> bit) & 1u;
      const uint64_t bb = __ballot(on);
      same &= on ? bb : ~bb;
    }
    rank[i] = static_cast<uint32_t>(__popcll(same & lt));
    if (rank[i] == 0) cnt[key[i]][i * kWaves + wave] = static_cast<uint16_t>(__popcll(same));
  }
  __syncthreads();
  // per bucket: counts before each step (in place), total, and the bucket
  // starts by a block scan of the totals (thread t: bucket t).  Dropped
  // positions are not written, so their bucket needs no prefix.
  auto prefix_steps = [&](int b) {
    u32x4* wp = reinterpret_cast<u32x4*>(&cnt[b][0]);
    const u32x4 w0 = wp[0], w1 = wp[1];
    uint32_t run = 0;
    u32x4 o0, o1;
#pragma unroll
    for (int q = 0; q < 8; ++q) {  // two counts per 32-bit word
      const uint32_t x = q < 4 ? w0[q] : w1[q - 4];
      const uint32_t lo16 = run;
      run += x & 0xffffu;
      const uint32_t hi16 = run;
      run += x >> 16;
      const uint32_t packed = lo16 | (hi16 << 16);
      if (q < 4) o0[q] = packed; else o1[q - 4] = packed;
    }
    wp[0] = o0;
    wp[1] = o1;
    return run;
  };
  const uint32_t tot = t < NB ? prefix_steps(t) : 0u;
  const uint32_t inc = wave_incl_sum(tot);
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  uint32_t before = inc - tot;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) before += w < wave ? wsum[w] : 0u;  // loads in flight together
  if (t < NB) start[t] = before;
  if (t == THREADS - 1) start[NB] = before + tot;  // kept positions of the block
  __syncthreads();
  uint32_t* bs = bstart + (int64_t)blockIdx.x * (NB + 1);
  if (t < NB) bs[t] = start[t];
  if (t == THREADS - 1) bs[NB] = start[NB];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (key[i] == NB) continue;
    const uint32_t slot = start[key[i]] + cnt[key[i]][i * kWaves + wave] + rank[i];
    if constexpr (!ROWS) sorted_pos[b0 + slot] = static_cast<uint32_t>(b0 + i * THREADS + t);
    sorted_seg[b0 + slot] = static_cast<uint16_t>(v[i]);
    if constexpr (ROWS)
      sorted_row[b0 + slot] = static_cast<uint64_t>(iv[i]) < static_cast<uint64_t>(rows)
                                  ? static_cast<uint32_t>(iv[i]) : 0xffffffffu;
  }
}

// Row ids of bag positions from a global list of row ids (uint32; ids
// outside the table are 0xffffffff).
struct GlobalRows {
  const int32_t* rows;
  template <int K>
  __device__ __forceinline__ void operator()(int64_t (&at)[K], const bool (&)[K],
                                             int64_t (&idv)[K]) const {
#pragma unroll
    for (int t = 0; t < K; ++t) idv[t] = static_cast<int64_t>(static_cast<uint32_t>(rows[at[t]]));
  }
};

// Row ids of bag positions from LDS (the fused reduction's ranked list).
struct LdsIds {
  const uint32_t* rows;
  template <int K>
  __device__ __forceinline__ void operator()(int64_t (&at)[K], const bool (&)[K],
                                             int64_t (&idv)[K]) const {
#pragma unroll
    for (int t = 0; t < K; ++t) idv[t] = static_cast<int64_t>(rows[at[t]]);
  }
};

// FUSED: instead of perm and offsets for the bag kernel, the workgroup
// reduces its segments itself (bag_group, G lanes per segment, 16-byte row
// chunks, table below 2 GiB) into out[batch, dim].  Its list then holds row
// ids (from step 1), so the rows are one round trip away.  A range with
// more entries than the list holds ranks them into perm (row ids, in its
// own slots) and reduces through it.
template <int G, bool MEAN, bool FUSED>
__global__ __launch_bounds__(kTlThreads) void seg_range_kernel(
    const uint32_t* __restrict__ sorted_val, const uint16_t* __restrict__ sorted_seg,
    const uint32_t* __restrict__ bstart, int nblk, int batch, int S, int sbits,
    int64_t* __restrict__ offsets, int32_t* __restrict__ perm, const float* __restrict__ data,
    int64_t rows, int64_t dim, float* __restrict__ out, int* __restrict__ status) {
  __shared__ uint32_t src[kTlMaxBlocks];        // sorted index of the range's first entry in block a
  __shared__ uint32_t excl[kTlMaxBlocks + 1];   // the range's entries in the blocks before a
  __shared__ uint32_t list_pos[kTlCap];         // the range's positions (FUSED: row ids), in order
  __shared__ uint8_t list_seg[kTlCap];          // ... and their segments less the range's first
  __shared__ uint32_t lrow[FUSED ? kTlCap : 1]; // FUSED: row ids ranked by segment
  __shared__ uint32_t sstart[kTlMaxS + 1];      // segment starts in the ranked list
  __shared__ uint16_t bmap[kTlCap];             // block of each list entry (gather)
  __shared__ uint32_t wcnt[kTlWaves][kTlMaxS];  // entries per wave slice and segment
  __shared__ uint32_t wpref[kTlWaves][kTlMaxS]; // next perm slot per wave slice and segment
  __shared__ uint32_t cursor[kTlMaxS];          // next perm slot per segment
  __shared__ uint32_t wsum[kTlWaves], wbelow[kTlWaves];
  __shared__ uint32_t total_s, base_all_s;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  const int g = blockIdx.x;
  const uint32_t lo = static_cast<uint32_t>(g) * S;
  const uint32_t ns = static_cast<uint32_t>(min(S, batch - static_cast<int>(lo)));

  // 1. the range's slice of every block: thread tid takes blocks
  //    [tid*per, tid*per + per); loads unconditional (block clamped)
  const int per = (nblk + kTlThreads - 1) / kTlThreads;
  uint32_t s0[kTlPer], cnt[kTlPer];
#pragma unroll
  for (int u = 0; u < kTlPer; ++u) {
    if (u < per) {
      const int a = min(tid * per + u, nblk - 1);
      const uint32_t* bs = bstart + (int64_t)a * (kTlBuckets + 1) + g;
      s0[u] = bs[0];
      cnt[u] = bs[1];
    }
  }
  uint32_t below = 0, mine = 0;
#pragma unroll
  for (int u = 0; u < kTlPer; ++u) {
    if (u < per) {
      const bool ok = tid * per + u < nblk;
      cnt[u] = ok ? cnt[u] - s0[u] : 0u;
      below += ok ? s0[u] : 0u;
      mine += cnt[u];
    }
  }
  // block scan of the per-thread entry counts; block sum of `below`
  uint32_t inc = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t x = __shfl_up(inc, off, 64);
    if (lane >= off) inc += x;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) below += __shfl_xor(below, off, 64);
  if (lane == 63) wsum[wave] = inc;
  if (lane == 0) wbelow[wave] = below;
  __syncthreads();
  uint32_t run = inc - mine;
  for (int w = 0; w < wave; ++w) run += wsum[w];
#pragma unroll
  for (int u = 0; u < kTlPer; ++u) {
    if (u < per) {
      const int a = tid * per + u;
      if (a < nblk) {
        src[a] = static_cast<uint32_t>(a) * kTlBlock + s0[u];
        excl[a] = run;
        run += cnt[u];
      }
    }
  }
  if (tid == kTlThreads - 1) {
    excl[nblk] = run;  // the last thread's running sum is the total
    total_s = run;
    uint32_t b = 0;
    for (int w = 0; w < kTlWaves; ++w) b += wbelow[w];
    base_all_s = b;
  }
  __syncthreads();
  const uint32_t total = total_s;

  // entries [c0, c0 + len) into the list (from `vals`: positions or row
  // ids): each thread marks its blocks' entries in bmap, then every thread
  // takes four entries (balanced, however the entries fall on the blocks),
  // all four loads in flight
  auto gather = [&](const uint32_t* __restrict__ vals, uint32_t c0, uint32_t len) {
#pragma unroll
    for (int u = 0; u < kTlPer; ++u) {
      if (u < per) {
        const int a = tid * per + u;
        if (a < nblk) {
          const uint32_t e0 = excl[a];
          const uint32_t hi_i = min(e0 + cnt[u], c0 + len);
          for (uint32_t i = max(e0, c0); i < hi_i; ++i) bmap[i - c0] = static_cast<uint16_t>(a);
        }
      }
    }
    __syncthreads();
    for (uint32_t i0 = 0; i0 < len; i0 += 4 * kTlThreads) {
      uint32_t e[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t i = min(i0 + q * kTlThreads + tid, len - 1);
        const int a = bmap[i];
        e[q] = src[a] + (c0 + i - excl[a]);
      }
      uint32_t p[4];
      uint16_t sg[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        p[q] = vals[e[q]];
        sg[q] = sorted_seg[e[q]];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t i = i0 + q * kTlThreads + tid;
        if (i < len) {
          list_pos[i] = p[q];
          list_seg[i] = static_cast<uint8_t>(sg[q] - lo);
        }
      }
    }
  };
  // lanes of this wave step holding the same segment
  auto match = [&](uint32_t seg_local, bool valid) {
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kTlMaxSBits; ++b) {
      if (b < sbits) {
        const bool on = (seg_local >> b) & 1u;
        const uint64_t bb = __ballot(on);
        same &= on ? bb : ~bb;
      }
    }
    return same;
  };
  auto slice = [&](uint32_t len, uint32_t* beg, uint32_t* end) {
    const uint32_t per_w = (len + kTlWaves - 1) / kTlWaves;
    *beg = wave * per_w;
    *end = min(len, *beg + per_w);
  };
  // wcnt[wave][s] += entries of segment s in this wave's slice of the list
  auto count_pass = [&](uint32_t len) {
    uint32_t beg, end;
    slice(len, &beg, &end);
    for (uint32_t k0 = beg; k0 < end; k0 += 64) {
      const uint32_t k = k0 + lane;
      const bool valid = k < end;
      const uint32_t s = valid ? list_seg[k] : 0u;
      const uint64_t same = match(s, valid);
      const uint32_t c = static_cast<uint32_t>(__popcll(same));
      if (valid && static_cast<uint32_t>(__popcll(same & lt)) + 1 == c) wcnt[wave][s] += c;
    }
  };
  // wpref[w][s] = cursor[s] + the entries of s in the slices before w;
  // returns the cursor after this list (for the last slice's threads)
  auto prefix_pass = [&]() {
    uint32_t r = 0;
    if (static_cast<uint32_t>(lane) < ns) {
      r = cursor[lane];
      for (int q = 0; q < wave; ++q) r += wcnt[q][lane];
      wpref[wave][lane] = r;
      r += wcnt[wave][lane];
    }
    return r;
  };
  // to_lds: the list's row ids into lrow (slots less the range's start);
  // else its values (positions, or FUSED: row ids) into perm
  auto write_pass = [&](uint32_t len, bool to_lds) {
    uint32_t beg, end;
    slice(len, &beg, &end);
    const uint32_t base_all = base_all_s;
    for (uint32_t k0 = beg; k0 < end; k0 += 64) {
      const uint32_t k = k0 + lane;
      const bool valid = k < end;
      const uint32_t s = valid ? list_seg[k] : 0u;
      const uint64_t same = match(s, valid);
      if (valid) {
        const uint32_t rank = static_cast<uint32_t>(__popcll(same & lt));
        const uint32_t c = static_cast<uint32_t>(__popcll(same));
        const uint32_t slot = wpref[wave][s] + rank;
        if (FUSED && to_lds)
          lrow[slot - base_all] = list_pos[k];
        else
          perm[slot] = static_cast<int32_t>(list_pos[k]);
        if (rank + 1 == c) wpref[wave][s] += c;
      }
    }
  };
  // segment counts (summed over the wave slices) -> offsets and cursors
  auto seg_offsets = [&]() {
    uint32_t c = 0;
    if (static_cast<uint32_t>(lane) < ns)
      for (int q = 0; q < kTlWaves; ++q) c += wcnt[q][lane];
    uint32_t sc = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t x = __shfl_up(sc, off, 64);
      if (lane >= off) sc += x;
    }
    const uint32_t base_all = base_all_s;
    const uint32_t start = base_all + sc - c;
    if (static_cast<uint32_t>(lane) < ns) {
      cursor[lane] = start;
      sstart[lane] = sc - c;
      if (!FUSED) offsets[lo + lane] = start;
    }
    if (lane == 63) {
      sstart[ns] = sc;
      if (!FUSED && lo + ns == static_cast<uint32_t>(batch)) offsets[batch] = base_all + sc;
    }
  };
  // FUSED: every segment of the range, G lanes each, from row ids fetched
  // by `ids` at list indices base + sstart[s] .. base + sstart[s + 1]
  auto reduce = [&](auto ids, uint32_t base) {
    if constexpr (FUSED) {
      constexpr int kGroups = kTlThreads / G;
      bool bad = false;
      for (uint32_t s = tid / G; s < ns; s += kGroups)
        bad |= bag_group<G, 4, MEAN, true>(data, rows, dim, base + sstart[s], base + sstart[s + 1],
                                           ids, out + static_cast<int64_t>(lo + s) * dim);
      if (bad) atomicOr(status, 1);
    }
  };
  uint32_t* wflat = &wcnt[0][0];

  if (total <= static_cast<uint32_t>(kTlCap)) {
    // the usual case: one list; its count pass also gives the segment sizes
    wflat[tid] = 0;
    gather(sorted_val, 0, total);
    __syncthreads();
    count_pass(total);
    __syncthreads();
    if (wave == 0) seg_offsets();
    __syncthreads();
    prefix_pass();
    __syncthreads();
    write_pass(total, true);
    if constexpr (FUSED) {
      __syncthreads();
      reduce(LdsIds{lrow}, 0u);
    }
    return;
  }
  // more entries than the list holds: chunks in order; a counting sweep
  // gives the segment sizes, a writing sweep carries the cursors
  wflat[tid] = 0;
  for (int sweep = 0; sweep < 2; ++sweep) {
    if (sweep == 1) {
      __syncthreads();
      if (wave == 0) seg_offsets();
    }
    for (uint32_t c0 = 0; c0 < total; c0 += kTlCap) {
      const uint32_t len = min(total - c0, static_cast<uint32_t>(kTlCap));
      __syncthreads();  // the previous chunk's readers of the list and wcnt are done
      if (sweep == 1) wflat[tid] = 0;
      gather(sorted_val, c0, len);
      __syncthreads();
      count_pass(len);
      if (sweep == 1) {
        __syncthreads();
        const uint32_t next = prefix_pass();
        __syncthreads();
        if (wave == kTlWaves - 1 && static_cast<uint32_t>(lane) < ns) cursor[lane] = next;
        write_pass(len, false);
      }
    }
  }
  if constexpr (FUSED) {
    // this workgroup's perm entries are read back by other lanes of it
    __threadfence();
    __syncthreads();
    reduce(GlobalRows{perm}, base_all_s);
  }
}

// ---------------------------------------------------------------------------
// Fused second step with one wave per segment range (the usual path of the
// two-level sort when the rows are reduced in place; blocks of 1024
// positions sorted into NB ranges by seg_block_sort_kernel<.., 1024, 1, NB>).
// A single wave has no cross-wave barriers, and its stable ranking keeps the
// per-segment counters in registers: lane s holds segment s's counter, and
// every wave step of 64 list entries builds, from four ballots, both the
// mask of each entry's segment (its rank: the entries of that segment in
// lower lanes) and the mask of segment `lane` (the counter update).
//   1. slices: lane l takes blocks [l*per, l*per + per); a wave scan of the
//      slice lengths gives each block's place in the range's list.
//   2. gather: the list (row ids and segments, position order) into LDS,
//      balanced over the lanes however the entries fall on the blocks.
//   3. count pass, exclusive scan over the segment lanes (segment starts),
//      write pass: row ids ranked by segment.
//   4. reduction: G lanes per segment (bag_group), rows in ranked order.
// A range with more than kRwCap entries is ranked chunk by chunk (a count
// sweep, then a write sweep carrying the counters) into perm, from which it
// is reduced.
// ---------------------------------------------------------------------------
constexpr int kRwBuckets = 1024;                // segment ranges (one wave each)
constexpr int kRwKeyBits = 11;                  // keys 0..kRwBuckets
constexpr int kRwBlock = 1024;                  // positions per block (1024 threads x 1)
constexpr int kRwMaxBlocks = 1024;              // up to 1 Mi positions
constexpr int kRwPer = kRwMaxBlocks / 64;       // blocks per lane
constexpr int kRwCap = 2048;                    // the list (LDS)
constexpr int kRwMaxS = 16;                     // segments per range (one per lane)
constexpr int kRwSBits = 4;                     // bits of a segment's place in its range
static_assert(kRwBlock == kTlBlock, "both steps share the block layout of the sorted arrays");
static_assert(kCsMaxSegments <= int64_t(kRwBuckets) * kRwMaxS, "segment ranges");

// Workgroup b's range when consecutive workgroups go to the 8 XCDs in turn:
// each XCD takes a run of consecutive ranges, whose slices of every block
// are adjacent in memory.
__device__ __forceinline__ int xcd_run(int b, int n) {
  const int per = n / 8, rem = n % 8, x = b % 8, k = b / 8;
  return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + k;
}

// PER: blocks per lane at most (nblk <= 64 * PER).
template <int G, bool MEAN, int NB, int PER>
__global__ __launch_bounds__(64) void seg_range_wave_kernel(
    const uint32_t* __restrict__ sorted_row, const uint16_t* __restrict__ sorted_seg,
    const uint32_t* __restrict__ bstart, int nblk, int batch, int S, int32_t* __restrict__ perm, const float* __restrict__ data, int64_t rows, int64_t dim,
    float* __restrict__ out, int* __restrict__ status) {
  __shared__ uint32_t src[kRwMaxBlocks];       // sorted index of the range's first entry in block a
  __shared__ uint32_t excl[kRwMaxBlocks + 1];  // the range's entries in the blocks before a
  __shared__ uint32_t list_row[kRwCap];        // the range's row ids, in position order
  __shared__ uint8_t list_seg[kRwCap];         // ... and their segments less the range's first
  __shared__ uint16_t bmap[kRwCap];            // block of each list entry (gather)
  __shared__ uint32_t lrow[kRwCap];            // row ids ranked by segment
  __shared__ uint32_t sstart[kRwMaxS + 1];     // segment starts in the ranked list

  const int lane = threadIdx.x;
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  const int g = xcd_run(blockIdx.x, gridDim.x);
  const uint32_t lo = static_cast<uint32_t>(g) * S;
  const uint32_t ns = static_cast<uint32_t>(min(S, batch - static_cast<int>(lo)));

  // 1. slices (loads unconditional: block clamped)
  const int per = (nblk + 63) / 64;
  uint32_t s0[PER], cnt[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    if (u < per) {
      const int a = min(lane * per + u, nblk - 1);
      const uint32_t* bs = bstart + (int64_t)a * (NB + 1) + g;
      s0[u] = bs[0];
      cnt[u] = bs[1];
    }
  }
  uint32_t below = 0, mine = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    if (u < per) {
      const bool ok = lane * per + u < nblk;
      cnt[u] = ok ? cnt[u] - s0[u] : 0u;
      below += ok ? s0[u] : 0u;
      mine += cnt[u];
    }
  }
  const uint32_t inc = wave_incl_sum(mine);
  const uint32_t total = lane63(inc);
  const uint32_t base_all = lane63(wave_incl_sum(below));  // this range's first slot in perm
  const uint32_t first = inc - mine;  // this lane's first list entry
  uint32_t run = first;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    if (u < per) {
      const int a = lane * per + u;
      if (a < nblk) {
        src[a] = static_cast<uint32_t>(a) * kRwBlock + s0[u];
        excl[a] = run;
        run += cnt[u];
      }
    }
  }
  __syncthreads();

  // 2. list entries [c0, c0 + len) into LDS (row ids and local segments)
  auto gather = [&](uint32_t c0, uint32_t len) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      if (u < per) {
        const int a = lane * per + u;
        if (a < nblk) {
          const uint32_t e0 = excl[a];
          const uint32_t hi_i = min(e0 + cnt[u], c0 + len);
          for (uint32_t i = max(e0, c0); i < hi_i; ++i) bmap[i - c0] = static_cast<uint16_t>(a);
        }
      }
    }
    __syncthreads();
    for (uint32_t i0 = 0; i0 < len; i0 += 4 * 64) {
      uint32_t e[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t i = min(i0 + q * 64 + lane, len - 1);
        const int a = bmap[i];
        e[q] = src[a] + (c0 + i - excl[a]);
      }
      uint32_t r[4];
      uint16_t sg[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        r[q] = sorted_row[e[q]];
        sg[q] = sorted_seg[e[q]];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t i = i0 + q * 64 + lane;
        if (i < len) {
          list_row[i] = r[q];
          list_seg[i] = static_cast<uint8_t>(sg[q] - lo);
        }
      }
    }
    __syncthreads();
  };
  // the step's ballots of the segment bits: masks of segment `s` among the
  // valid entries
  // (all kRwSBits bits: a range's segments past S have no entries, so
  // their masks are empty)
  struct Step {
    uint64_t valid, bit[kRwSBits];
  };
  auto step_ballots = [&](uint32_t s, bool valid) {
    Step st;
    st.valid = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRwSBits; ++b) st.bit[b] = __ballot(valid && ((s >> b) & 1u));
    return st;
  };
  auto seg_mask = [&](const Step& st, uint32_t s) {
    uint64_t m = st.valid;
#pragma unroll
    for (int b = 0; b < kRwSBits; ++b) m &= ((s >> b) & 1u) ? st.bit[b] : ~st.bit[b];
    return m;
  };
  // 3a. lane s += the entries of segment s among list entries [0, len)
  auto count_pass = [&](uint32_t len, uint32_t* c_s) {
    for (uint32_t k0 = 0; k0 < len; k0 += 64) {
      const uint32_t k = k0 + lane;
      const bool valid = k < len;
      const Step st = step_ballots(valid ? list_seg[k] : 0u, valid);
      *c_s += static_cast<uint32_t>(__popcll(seg_mask(st, static_cast<uint32_t>(lane))));
    }
  };
  // 3c. each entry to its segment's cursor (lane s holds segment s's) plus
  // its rank; to_lds: into lrow (slots relative to the range), else perm
  auto write_pass = [&](uint32_t len, uint32_t* cur_s, bool to_lds) {
    for (uint32_t k0 = 0; k0 < len; k0 += 64) {
      const uint32_t k = k0 + lane;
      const bool valid = k < len;
      const uint32_t s = valid ? list_seg[k] : 0u;
      const Step st = step_ballots(s, valid);
      const uint32_t rank = static_cast<uint32_t>(__popcll(seg_mask(st, s) & lt));
      const uint32_t base = static_cast<uint32_t>(__shfl(static_cast<int>(*cur_s), static_cast<int>(s), 64));
      if (valid) {
        if (to_lds)
          lrow[base + rank] = list_row[k];
        else
          perm[base + rank] = static_cast<int32_t>(list_row[k]);
      }
      *cur_s += static_cast<uint32_t>(__popcll(seg_mask(st, static_cast<uint32_t>(lane))));
    }
  };
  // 3b. segment starts (relative to the range) from the counts of lanes < ns
  // (a lane at or past ns matched the segment its low kRwSBits bits name)
  auto seg_starts = [&](uint32_t c_s) {
    if (static_cast<uint32_t>(lane) >= ns) c_s = 0;
    const uint32_t sc = wave_incl_sum(c_s);
    if (static_cast<uint32_t>(lane) < ns) sstart[lane] = sc - c_s;
    if (lane == 63) sstart[ns] = sc;
    return sc - c_s;
  };
  // 4. G lanes per segment; `ids` gives row ids at list index base + j
  auto reduce = [&](auto ids, uint32_t base) {
    constexpr int kGroups = 64 / G;
    bool bad = false;
    for (uint32_t s = lane / G; s < ns; s += kGroups)
      bad |= bag_group<G, 4, MEAN, true>(data, rows, dim, base + sstart[s], base + sstart[s + 1],
                                         ids, out + static_cast<int64_t>(lo + s) * dim);
    if (bad) atomicOr(status, 1);
  };

  // The common case: at most two blocks and four entries per lane.  Each
  // lane loads its own entries (no block map) and keeps them in registers;
  // the list order is lane-major, so an entry's rank within its segment is
  // the entries of that segment in lower lanes (four ballot sets, one per
  // register slot) plus those in lower slots of its own lane.  Only the
  // ranked row ids go to LDS.
  auto rank_direct = [&]() {
    const uint32_t c0 = cnt[0];
    const uint32_t src0 = static_cast<uint32_t>(min(lane * per, nblk - 1)) * kRwBlock + s0[0];
    const uint32_t src1 = per > 1 ? static_cast<uint32_t>(min(lane * per + 1, nblk - 1)) * kRwBlock + s0[1]
                                  : src0;
    uint32_t e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t jj = static_cast<uint32_t>(j) < mine ? static_cast<uint32_t>(j) : 0u;
      e[j] = jj < c0 ? src0 + jj : src1 + (jj - c0);
    }
    uint32_t r[4];
    uint16_t sg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r[j] = sorted_row[e[j]];
      sg[j] = sorted_seg[e[j]];
    }
    uint32_t ls[4];
    bool ok[4];
    Step st[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ok[j] = static_cast<uint32_t>(j) < mine;
      ls[j] = ok[j] ? static_cast<uint32_t>(sg[j] - lo) : 0u;
      st[j] = step_ballots(ls[j], ok[j]);
    }
    uint32_t c_lane = 0;  // entries of segment `lane`
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c_lane += static_cast<uint32_t>(__popcll(seg_mask(st[j], static_cast<uint32_t>(lane))));
    const uint32_t cur = seg_starts(c_lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t rank = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rank += static_cast<uint32_t>(__popcll(seg_mask(st[i], ls[j]) & lt));
        if (i < j) rank += (ok[i] && ls[i] == ls[j]) ? 1u : 0u;
      }
      const uint32_t base = static_cast<uint32_t>(__shfl(static_cast<int>(cur), static_cast<int>(ls[j]), 64));
      if (ok[j] && base + rank < static_cast<uint32_t>(kRwCap)) lrow[base + rank] = r[j];
    }
    __syncthreads();
  };

  uint32_t c_s = 0;
  if (total <= static_cast<uint32_t>(kRwCap)) {
    if (per <= 2 && __ballot(mine > 4) == 0) {
      rank_direct();
      reduce(LdsIds{lrow}, 0u);
      return;
    }
    gather(0, total);
    count_pass(total, &c_s);
    uint32_t cur_s = seg_starts(c_s);
    write_pass(total, &cur_s, true);
    __syncthreads();
    reduce(LdsIds{lrow}, 0u);
    return;
  }
  for (uint32_t c0 = 0; c0 < total; c0 += kRwCap) {
    const uint32_t len = min(total - c0, static_cast<uint32_t>(kRwCap));
    gather(c0, len);
    count_pass(len, &c_s);
    __syncthreads();  // the list is read again by the next chunk's gather
  }
  uint32_t cur_s = base_all + seg_starts(c_s);
  for (uint32_t c0 = 0; c0 < total; c0 += kRwCap) {
    const uint32_t len = min(total - c0, static_cast<uint32_t>(kRwCap));
    gather(c0, len);
    write_pass(len, &cur_s, false);
    __syncthreads();
  }
  // this wave's perm entries are read back by its other lanes
  __threadfence();
  __syncthreads();
  reduce(GlobalRows{perm}, base_all);
}

// Sort keys: the segment id, or `batch` for ids outside [0, batch), which
// then sort after every kept position.
__global__ void make_keys_kernel(const int64_t* __restrict__ seg, int64_t stride, int64_t n,
                                 int64_t batch, uint32_t* __restrict__ keys,
                                 int32_t* __restrict__ vals) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t v = seg[i * stride];
  keys[i] = static_cast<uint32_t>(v >= 0 && v < batch ? v : batch);
  vals[i] = static_cast<int32_t>(i);
}

// ---------------------------------------------------------------------------
// sparse_embedding2 and __pooling
// ---------------------------------------------------------------------------
template <typename IdxT>
__global__ __launch_bounds__(kThreads) void sparse_embedding2_kernel(
    const float* __restrict__ table, int64_t rows, int64_t dim, const IdxT* __restrict__ ids,
    int64_t n, int64_t fallback, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n * dim) return;
  const int64_t i = t / dim, d = t % dim;
  const int64_t id = static_cast<int64_t>(ids[i]);
  const bool valid = id >= 0 && id < rows;
  const float mask = valid ? 1.0f : 0.0f;
  out[t] = table[(valid ? id : fallback) * dim + d] * mask;
}

// Rows of dim % 4 == 0 with 16-byte aligned table and output: G lanes per
// id (G = dim/4 rounded up to a power of two, at most 64), one 16-byte load
// and store per lane per chunk of 4*G floats.
template <typename IdxT, int G>
__global__ __launch_bounds__(kThreads) void sparse_embedding2_vec_kernel(
    const float* __restrict__ table, int64_t rows, int64_t dim, const IdxT* __restrict__ ids,
    int64_t n, int64_t fallback, float* __restrict__ out) {
  const int g = threadIdx.x & (G - 1);
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / G;
  if (i >= n) return;
  const int64_t id = static_cast<int64_t>(ids[i]);
  const bool valid = id >= 0 && id < rows;
  const float mask = valid ? 1.0f : 0.0f;
  const float* src = table + (valid ? id : fallback) * dim;
  float* dst = out + i * dim;
  for (int64_t c = 4 * g; c < dim; c += 4 * G) store_row<4>(dst + c, load_row<4>(src + c) * mask);
}

// __pooling with n % 4 == 0, 16-byte aligned `gathered` below 2 GiB: G lanes
// per output row (G = n/4 rounded up to a power of two, at most 64), each
// lane summing 4 columns in j order.  Positions are taken in rounds of
// kGroupRound: the lanes fetch the round's ids (distinct ids per lane,
// coalesced) and turn them into byte offsets, and the round's row loads are
// issued together, offsets broadcast inside the group.  Positions with
// id <= 0 read zeros past the buffer's range check (no traffic), which add
// nothing to the +0-seeded sums.  The count of ids > 0 is exact (k < 2^24),
// as the reference's float count is.
template <int G>
__global__ __launch_bounds__(kThreads) void pooling_vec_kernel(
    const int64_t* __restrict__ ids, const float* __restrict__ gathered, int64_t m, int64_t k,
    int64_t n, int64_t ss0, int64_t ss1, int64_t ss2, int64_t sl0, int64_t sl1, int64_t sl2,
    float* __restrict__ out) {
  typedef typename VecT<4>::type V;
  constexpr int kPer = (kGroupRound + G - 1) / G;
  const int g = threadIdx.x & (G - 1);
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / G;
  if (i >= m) return;
  const int64_t* row_ids = ids + i * k;
  int cnt = 0;
  for (int64_t j = g; j < k; j += G) cnt += row_ids[j] > 0 ? 1 : 0;
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, G);
  const float red = static_cast<float>(cnt);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(gathered), 0, static_cast<int>(m * k * n * 4), kRawBufferFlags);
  const bool row_in = i >= ss0 && i < sl0;
  const int64_t j0 = ss1 > 0 ? ss1 : 0;
  const int64_t j1 = sl1 < k ? sl1 : k;
  const uint32_t row_base = static_cast<uint32_t>(i * k * n * 4);
  const uint32_t step = static_cast<uint32_t>(n * 4);
  // Every lane of the group runs every column chunk (lanes past n load
  // nothing and store nothing), so the broadcasts never read a lane that
  // has left the loop.
  const int64_t chunks = (n + 4 * G - 1) / (4 * G);
  for (int64_t cc = 0; cc < chunks; ++cc) {
    const int64_t c = cc * 4 * G + 4 * g;
    const bool active = c < n;
    V sum = V(0.0f);
    if (row_in) {
      for (int64_t jb = j0; jb < j1; jb += kGroupRound) {
        uint32_t off[kPer];
#pragma unroll
        for (int t = 0; t < kPer; ++t) {
          const int64_t j = jb + g + G * t;
          const int64_t id = j < j1 ? row_ids[j] : 0;
          off[t] = id > 0 ? row_base + static_cast<uint32_t>(j) * step : kMaskedOff;
        }
        V v[kGroupRound];
        static_for([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          const uint32_t o = group_bcast<G, u % G>(off[u / G]);
          v[u] = buffer_row<4>(rsrc, (o == kMaskedOff || !active)
                                         ? kMaskedOff
                                         : o + static_cast<uint32_t>(c * 4));
        }, std::make_integer_sequence<int, kGroupRound>{});
#pragma unroll
        for (int u = 0; u < kGroupRound; ++u) sum += v[u];
      }
    }
    V res;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t p = c + e;
      const float s = (p >= ss2 && p < sl2) ? sum[e] : 0.0f;
      res[e] = red == 0.0f ? 0.0f : s / red;
    }
    if (active) store_row<4>(out + i * n + c, res);
  }
}

// __pooling for rows of k <= R positions (R = 16, 32 or 48): one round.  The
// row's ids are loaded once and give both the count of ids > 0 and the row
// offsets, and all R row loads of a lane are issued before the first add, so
// the kernel is one id round trip and one row round trip (the multi-round
// kernel above reloads the ids per round and per column chunk).  Positions
// past k, outside the slice or with id <= 0 read past the buffer range and
// add +0.0f, which leaves the in-order sum unchanged.
// (At most R*G/64 waves per bag row group run per SIMD on the benchmark
// shapes, so the kernel asks for 1-2 waves per SIMD and the registers to
// keep every row load in flight.)
template <int G, int R>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void
pooling_round_kernel(
    const int64_t* __restrict__ ids, const float* __restrict__ gathered, int64_t m, int64_t k,
    int64_t n, int64_t ss0, int64_t ss1, int64_t ss2, int64_t sl0, int64_t sl1, int64_t sl2,
    float* __restrict__ out) {
  typedef typename VecT<4>::type V;
  constexpr int kPer = (R + G - 1) / G;
  const int g = threadIdx.x & (G - 1);
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / G;
  if (i >= m) return;
  const int64_t* row_ids = ids + i * k;
  const bool row_in = i >= ss0 && i < sl0;
  const int64_t j0 = ss1 > 0 ? ss1 : 0;
  const int64_t j1 = sl1 < k ? sl1 : k;
  const uint32_t row_base = static_cast<uint32_t>(i * k * n * 4);
  const uint32_t step = static_cast<uint32_t>(n * 4);
  int cnt = 0;
  uint32_t off[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int j = g + G * t;
    const int64_t id_c = row_ids[j < k ? j : k - 1];  // unconditional: one round trip
    const int64_t id = j < k ? id_c : 0;
    cnt += id > 0 ? 1 : 0;
    off[t] = (row_in && id > 0 && j >= j0 && j < j1) ? row_base + static_cast<uint32_t>(j) * step
                                                     : kMaskedOff;
  }
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, G);
  const float red = static_cast<float>(cnt);
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(gathered), 0, static_cast<int>(m * k * n * 4), kRawBufferFlags);
  // every lane runs every column chunk (see pooling_vec_kernel)
  const int64_t chunks = (n + 4 * G - 1) / (4 * G);
  for (int64_t cc = 0; cc < chunks; ++cc) {
    const int64_t c = cc * 4 * G + 4 * g;
    const bool active = c < n;
    V v[R];
    static_for([&](auto uc) {
      constexpr int u = decltype(uc)::value;
      const uint32_t o = group_bcast<G, u % G>(off[u / G]);
      v[u] = buffer_row<4>(rsrc, (o == kMaskedOff || !active) ? kMaskedOff
                                                              : o + static_cast<uint32_t>(c * 4));
    }, std::make_integer_sequence<int, R>{});
    V sum = V(0.0f);
#pragma unroll
    for (int u = 0; u < R; ++u) sum += v[u];
    V res;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t p = c + e;
      const float s = (p >= ss2 && p < sl2) ? sum[e] : 0.0f;
      res[e] = red == 0.0f ? 0.0f : s / red;
    }
    if (active) store_row<4>(out + i * n + c, res);
  }
}

__global__ __launch_bounds__(kThreads) void pooling_kernel(
    const int64_t* __restrict__ ids, const float* __restrict__ gathered, int64_t m, int64_t k,
    int64_t n, int64_t ss0, int64_t ss1, int64_t ss2, int64_t sl0, int64_t sl1, int64_t sl2,
    float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= m * n) return;
  const int64_t i = t / n, p = t % n;
  const int64_t* row_ids = ids + i * k;
  float red = 0.0f;
  for (int64_t j = 0; j < k; ++j) red += row_ids[j] > 0 ? 1.0f : 0.0f;
  float sum = 0.0f;
  const bool in_rows = i >= ss0 && i < sl0 && p >= ss2 && p < sl2;
  if (in_rows) {
    const int64_t j0 = ss1 > 0 ? ss1 : 0;
    const int64_t j1 = sl1 < k ? sl1 : k;
    for (int64_t j = j0; j < j1; ++j)
      if (row_ids[j] > 0) sum += gathered[(i * k + j) * n + p];
  }
  out[t] = red == 0.0f ? 0.0f : sum / red;
}

__global__ void widen_i32_kernel(const int32_t* __restrict__ src, int64_t n,
                                 int64_t* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

__global__ void nz_flag_kernel(const float* __restrict__ dense, int64_t count,
                               int32_t* __restrict__ flags) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < count) flags[i] = dense[i] != 0.0f ? 1 : 0;  // NaN counts as nonzero
}

// Writes the p-th listed value for p < cap only: a caller whose buffers hold
// fewer values than the flags list gets no write past them (the host then
// reports the count mismatch).
__global__ void nz_write_kernel(const float* __restrict__ dense, int64_t count, int64_t dim,
                                const int64_t* __restrict__ seg_of_row, int one_d,
                                const int32_t* __restrict__ flags,
                                const int32_t* __restrict__ incl, int64_t cap,
                                int32_t* __restrict__ out_idx, float* __restrict__ out_val) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= count || !flags[i]) return;
  const int64_t p = incl[i] - 1, r = i / dim;
  if (p >= cap) return;
  const int32_t seg = static_cast<int32_t>(seg_of_row[r]);
  if (one_d) {
    out_idx[p] = seg;
  } else {
    out_idx[2 * p] = seg;
    out_idx[2 * p + 1] = static_cast<int32_t>(i - r * dim);
  }
  out_val[p] = dense[i];
}

}  // namespace

int launch_bag(const BagArgs& a, hipStream_t s) {
  ANNC_REQUIRE(a.rows < static_cast<int64_t>(kNoRow), "tables of 2^32-1 rows or more are not supported");
  ANNC_REQUIRE(a.dim < (int64_t(1) << 29), "embedding dim must be below 2^29");
  return a.ids_is_64 ? launch_bag_idx<int64_t>(a, s) : launch_bag_idx<int32_t>(a, s);
}

int segment_scan(hipStream_t s, const int64_t* seg, int64_t stride, int64_t n, int64_t* min_out,
                 int64_t* max_out, bool* sorted) {
  *min_out = LLONG_MAX;
  *max_out = LLONG_MIN;
  *sorted = true;
  if (n <= 0) return ANNC_OK;
  // up to 256 blocks of 4 waves; their records are combined here
  constexpr int kMaxBlocks = 256;
  const int blocks = (int)std::min<int64_t>(kMaxBlocks, ceil_div(n, 4 * kThreads));
  void* ws = stream_workspace(s, sizeof(long long) * 3 * kMaxBlocks);
  if (!ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  long long* part = static_cast<long long*>(ws);
  hipLaunchKernelGGL(seg_scan_kernel, dim3(blocks), dim3(kThreads), 0, s, seg, stride, n, part);
  ANNC_HIP_TRY(hipGetLastError());
  long long host[3 * kMaxBlocks];
  const int rc = read_back(s, {{host, part, sizeof(long long) * 3 * blocks}});
  if (rc != ANNC_OK) return rc;
  for (int b = 0; b < blocks; ++b) {
    *min_out = std::min<int64_t>(*min_out, host[3 * b]);
    *max_out = std::max<int64_t>(*max_out, host[3 * b + 1]);
    if (host[3 * b + 2]) *sorted = false;
  }
  return ANNC_OK;
}

namespace {
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
}  // namespace

int segment_reduce_plan(int64_t n, int64_t batch, int sorted_hint, hipStream_t s, SegPlan* plan) {
  ANNC_REQUIRE(n < (1ll << 31) - 1, "too many indices");
  ANNC_REQUIRE(batch < (1ll << 32), "too many segments");
  *plan = SegPlan{};
  const size_t off_bytes = align256(sizeof(int64_t) * (size_t)(batch + 1));
  if (sorted_hint == 1) {
    plan->path = SegPlan::kSorted;  // no workspace
    return ANNC_OK;
  }
  const int64_t tblk = std::max<int64_t>(1, ceil_div(n, kTlBlock));
  if (batch <= kCsMaxSegments && tblk <= kTlMaxBlocks) {
    plan->path = SegPlan::kTwoLevel;
    const size_t m = (size_t)(tblk * kTlBlock);
    // sorted positions (or row ids), segments, bucket starts (kRwBuckets
    // ranges for the one-wave step, which takes up to kRwMaxBlocks blocks),
    // offsets, perm
    const int64_t nb = tblk <= kRwMaxBlocks ? kRwBuckets : kTlBuckets;
    plan->bytes = align256(sizeof(uint32_t) * m) + align256(sizeof(uint16_t) * m) +
                  align256(sizeof(uint32_t) * (size_t)(tblk * (nb + 1))) + off_bytes +
                  align256(sizeof(int32_t) * (size_t)std::max<int64_t>(n, 1));
    return ANNC_OK;
  }
  const int64_t nblk = ceil_div(n, kCsBlock);
  if (batch <= kCsMaxSegments && nblk * batch <= (int64_t(1) << 24)) {
    plan->path = SegPlan::kCounting;
    const size_t hb = align256(sizeof(uint32_t) * (size_t)std::max<int64_t>(nblk * batch, 1));
    const size_t tb = align256(sizeof(uint32_t) * (size_t)batch);
    const size_t pb = align256(sizeof(int32_t) * (size_t)std::max<int64_t>(n, 1));
    plan->bytes = 2 * hb + tb + off_bytes + pb;
    return ANNC_OK;
  }
  plan->path = SegPlan::kRadix;
  int end_bit = 1;
  while (end_bit < 32 && (1ull << end_bit) <= (uint64_t)batch) ++end_bit;  // batch fits too
  const size_t temp_bytes = radix_sort_temp_bytes(n);
  const size_t nk = align256(sizeof(uint32_t) * (size_t)std::max<int64_t>(n, 1));
  plan->end_bit = end_bit;
  plan->temp_bytes = temp_bytes;
  plan->bytes = 4 * nk + off_bytes + align256(temp_bytes);
  return ANNC_OK;
}

int segment_reduce_run(hipStream_t s, const float* data, int64_t rows, int64_t dim,
                       const void* indices, int indices_is_64, const int64_t* seg, int64_t stride,
                       int64_t n, int combiner, int64_t batch, float* out, const SegPlan& plan,
                       void* workspace, int* status) {
  if (batch <= 0) return ANNC_OK;
  BagArgs a{};
  a.table = data;
  a.rows = rows;
  a.dim = dim;
  a.ids = indices;
  a.ids_is_64 = indices_is_64;
  a.num_bags = batch;
  a.combiner = combiner;
  a.out = out;
  a.ldo = dim;
  a.status = status;
  char* ws = static_cast<char*>(workspace);
  const size_t off_bytes = align256(sizeof(int64_t) * (size_t)(batch + 1));

  if (plan.path == SegPlan::kSorted) {
    // one launch: segment boundaries found in LDS, no offsets array
    ANNC_REQUIRE(rows < static_cast<int64_t>(kNoRow), "tables of 2^32-1 rows or more are not supported");
    ANNC_REQUIRE(dim < (int64_t(1) << 29), "embedding dim must be below 2^29");
    return indices_is_64 ? launch_seg_sorted<int64_t>(a, seg, stride, n, s)
                         : launch_seg_sorted<int32_t>(a, seg, stride, n, s);
  }

  if (plan.path == SegPlan::kTwoLevel) {
    // block sort by segment range, then one workgroup per range, which
    // reduces its segments itself (fused) or writes perm for the bag kernel
    const int64_t tblk = std::max<int64_t>(1, ceil_div(n, kTlBlock));
    const size_t m = (size_t)(tblk * kTlBlock);
    uint32_t* sorted_pos = reinterpret_cast<uint32_t*>(ws);
    ws += align256(sizeof(uint32_t) * m);
    uint16_t* sorted_seg = reinterpret_cast<uint16_t*>(ws);
    ws += align256(sizeof(uint16_t) * m);
    uint32_t* bstart = reinterpret_cast<uint32_t*>(ws);
    const int64_t nb_alloc = tblk <= kRwMaxBlocks ? kRwBuckets : kTlBuckets;
    ws += align256(sizeof(uint32_t) * (size_t)(tblk * (nb_alloc + 1)));
    int64_t* offsets = reinterpret_cast<int64_t*>(ws);
    int32_t* perm = reinterpret_cast<int32_t*>(ws + off_bytes);
    // S segments per range: at most kTlBuckets ranges, S <= kTlMaxS
    const int S = static_cast<int>(std::max<int64_t>(1, ceil_div(batch, kTlBuckets)));
    int sbits = 0;
    while ((1 << sbits) < S) ++sbits;
    const int nb = n > 0 ? static_cast<int>(tblk) : 0;
    const dim3 rgrid((unsigned)ceil_div(batch, S));
    // fused: 16-byte row chunks and a table below 2 GiB (buffer loads)
    auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool fuse = n > 0 && dim % 4 == 0 && aligned16(data) && aligned16(out) &&
                      rows * dim * static_cast<int64_t>(sizeof(float)) < (int64_t(1) << 31);
    if (!fuse) {
      if (n > 0) {
        hipLaunchKernelGGL((seg_block_sort_kernel<int64_t, false, kTlThreads, kTlItems, kTlBuckets,
                                                kTlBucketBits>), dim3((unsigned)tblk),
                           dim3(kTlThreads), 0, s, seg, stride, n, static_cast<int>(batch), S,
                           static_cast<const int64_t*>(nullptr), rows, sorted_pos, sorted_seg,
                           static_cast<uint32_t*>(nullptr), bstart);
        ANNC_HIP_TRY(hipGetLastError());
      }
      hipLaunchKernelGGL((seg_range_kernel<4, false, false>), rgrid, dim3(kTlThreads), 0, s,
                         sorted_pos, sorted_seg, bstart, nb, static_cast<int>(batch), S, sbits,
                         offsets, perm, static_cast<const float*>(nullptr), rows, dim,
                         static_cast<float*>(nullptr), status);
      ANNC_HIP_TRY(hipGetLastError());
      a.offsets = offsets;
      a.perm = perm;
      return launch_bag(a, s);
    }
    // one wave per range (kRwBuckets ranges) up to kRwMaxBlocks blocks
    const bool wave = tblk <= kRwMaxBlocks;
    const int Sw = static_cast<int>(std::max<int64_t>(1, ceil_div(batch, kRwBuckets)));
    auto run_fused = [&](auto idx_tag) -> int {
      using IdxT = decltype(idx_tag);
      const IdxT* idx = static_cast<const IdxT*>(indices);
      // sorted_pos holds the row ids (ROWS)
      if (wave)
        hipLaunchKernelGGL((seg_block_sort_kernel<IdxT, true, kRwBlock, 1, kRwBuckets, kRwKeyBits>),
                           dim3((unsigned)tblk), dim3(kRwBlock), 0, s, seg, stride, n,
                           static_cast<int>(batch), Sw, idx, rows, static_cast<uint32_t*>(nullptr),
                           sorted_seg, sorted_pos, bstart);
      else
        hipLaunchKernelGGL((seg_block_sort_kernel<IdxT, true, kTlThreads, kTlItems, kTlBuckets,
                                                  kTlBucketBits>),
                           dim3((unsigned)tblk), dim3(kTlThreads), 0, s, seg, stride, n,
                           static_cast<int>(batch), S, idx, rows, static_cast<uint32_t*>(nullptr),
                           sorted_seg, sorted_pos, bstart);
      ANNC_HIP_TRY(hipGetLastError());
      const int64_t lanes = dim / 4;
      const bool mean = combiner == ANNC_COMBINER_MEAN;
      auto go = [&](auto g_tag) -> int {
        constexpr int G = decltype(g_tag)::value;
        if (wave) {
          // two blocks per lane up to 128 blocks (the usual case: no loops
          // over empty block slots), else up to kRwPer
          auto k = tblk <= 128 ? (mean ? seg_range_wave_kernel<G, true, kRwBuckets, 2>
                                       : seg_range_wave_kernel<G, false, kRwBuckets, 2>)
                               : (mean ? seg_range_wave_kernel<G, true, kRwBuckets, kRwPer>
                                       : seg_range_wave_kernel<G, false, kRwBuckets, kRwPer>);
          hipLaunchKernelGGL(k, dim3((unsigned)ceil_div(batch, Sw)), dim3(64), 0, s, sorted_pos,
                             sorted_seg, bstart, nb, static_cast<int>(batch), Sw, perm,
                             data, rows, dim, out, status);
        } else {
          auto k = mean ? seg_range_kernel<G, true, true> : seg_range_kernel<G, false, true>;
          hipLaunchKernelGGL(k, rgrid, dim3(kTlThreads), 0, s, sorted_pos, sorted_seg, bstart, nb,
                             static_cast<int>(batch), S, sbits, offsets, perm, data, rows, dim, out,
                             status);
        }
        ANNC_HIP_TRY(hipGetLastError());
        return ANNC_OK;
      };
      if (lanes <= 4) return go(std::integral_constant<int, 4>{});
      if (lanes <= 8) return go(std::integral_constant<int, 8>{});
      if (lanes <= 16) return go(std::integral_constant<int, 16>{});
      if (lanes <= 32) return go(std::integral_constant<int, 32>{});
      return go(std::integral_constant<int, 64>{});
    };
    return indices_is_64 ? run_fused(int64_t{}) : run_fused(int32_t{});
  }

  if (plan.path == SegPlan::kCounting) {
    // stable counting sort by segment (up to kCsMaxSegments segments)
    const int64_t nblk = ceil_div(n, kCsBlock);
    const size_t hb = align256(sizeof(uint32_t) * (size_t)std::max<int64_t>(nblk * batch, 1));
    const size_t tb = align256(sizeof(uint32_t) * (size_t)batch);
    uint32_t* H = reinterpret_cast<uint32_t*>(ws);
    uint32_t* P = reinterpret_cast<uint32_t*>(ws + hb);
    uint32_t* total = reinterpret_cast<uint32_t*>(ws + 2 * hb);
    int64_t* offsets = reinterpret_cast<int64_t*>(ws + 2 * hb + tb);
    int32_t* perm = reinterpret_cast<int32_t*>(ws + 2 * hb + tb + off_bytes);
    const int nb = static_cast<int>(batch);
    const size_t lds = sizeof(uint32_t) * (size_t)batch;
    if (n > 0) {
      hipLaunchKernelGGL(cs_hist_kernel, dim3((unsigned)nblk), dim3(kThreads), lds, s, seg, stride,
                         n, nb, H);
      ANNC_HIP_TRY(hipGetLastError());
    }
    hipLaunchKernelGGL(cs_prefix_kernel, dim3((unsigned)ceil_div(batch, 64)), dim3(1024), 0, s, H,
                       nb, static_cast<int>(nblk), P, total);
    ANNC_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(cs_offsets_kernel, dim3(1), dim3(1024), 0, s, total, nb, offsets);
    ANNC_HIP_TRY(hipGetLastError());
    if (n > 0) {
      hipLaunchKernelGGL(cs_scatter_kernel, dim3((unsigned)nblk), dim3(kThreads), lds, s, seg, stride, n,
                         nb, P, offsets, perm);
      ANNC_HIP_TRY(hipGetLastError());
    }
    a.offsets = offsets;
    a.perm = perm;
    return launch_bag(a, s);
  }

  // More segments: stable radix sort of (segment id, position), then CSR.
  const size_t nk = align256(sizeof(uint32_t) * (size_t)std::max<int64_t>(n, 1));
  uint32_t* keys_in = reinterpret_cast<uint32_t*>(ws);
  uint32_t* keys_out = reinterpret_cast<uint32_t*>(ws + nk);
  int32_t* vals_in = reinterpret_cast<int32_t*>(ws + 2 * nk);
  int32_t* vals_out = reinterpret_cast<int32_t*>(ws + 3 * nk);
  int64_t* offsets = reinterpret_cast<int64_t*>(ws + 4 * nk);
  void* temp = ws + 4 * nk + off_bytes;
  if (n > 0) {
    hipLaunchKernelGGL(make_keys_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0,
                       s, seg, stride, n, batch, keys_in, vals_in);
    ANNC_HIP_TRY(hipGetLastError());
    // sorted pairs end in keys_in / vals_in (the pointers follow the passes)
    const int rc = radix_sort_pairs(s, &keys_in, &keys_out, &vals_in, &vals_out, n, plan.end_bit,
                                    temp);
    if (rc != ANNC_OK) return rc;
  }
  hipLaunchKernelGGL(seg_bounds_kernel<uint32_t>, dim3((unsigned)ceil_div(n + 1, kThreads)),
                     dim3(kThreads), 0, s, keys_in, (int64_t)1, n, batch, offsets);
  ANNC_HIP_TRY(hipGetLastError());
  a.offsets = offsets;
  a.perm = vals_in;
  return launch_bag(a, s);
}

int segment_reduce(hipStream_t s, const float* data, int64_t rows, int64_t dim,
                   const void* indices, int indices_is_64, const int64_t* seg, int64_t stride,
                   int64_t n, int combiner, int64_t batch, float* out, int sorted_hint) {
  if (batch <= 0) return ANNC_OK;
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  SegPlan plan;
  int rc = segment_reduce_plan(n, batch, sorted_hint, s, &plan);
  if (rc != ANNC_OK) return rc;
  void* ws = plan.bytes ? stream_workspace(s, plan.bytes) : nullptr;
  if (plan.bytes && !ws) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  return segment_reduce_run(s, data, rows, dim, indices, indices_is_64, seg, stride, n, combiner,
                            batch, out, plan, ws, status);
}

namespace {

// Lanes per row for the vector kernels: dim/4 rounded up to a power of two,
// 1..64 (chunks of 4*64 floats beyond that).
int vec_group(int64_t dim4) {
  int g = 1;
  while (g < 64 && g < dim4) g <<= 1;
  return g;
}

template <typename IdxT>
int launch_se2_vec(hipStream_t s, const float* table, int64_t rows, int64_t dim, const IdxT* ids,
                   int64_t n, int64_t fallback, float* out) {
  const int g = vec_group(dim / 4);
  const dim3 grid((unsigned)ceil_div(n * g, kThreads));
  switch (g) {
#define ANNC_SE2(G)                                                                        \
  case G:                                                                                  \
    hipLaunchKernelGGL((sparse_embedding2_vec_kernel<IdxT, G>), grid, dim3(kThreads), 0, s, \
                       table, rows, dim, ids, n, fallback, out);                           \
    break;
    ANNC_SE2(1) ANNC_SE2(2) ANNC_SE2(4) ANNC_SE2(8) ANNC_SE2(16) ANNC_SE2(32) ANNC_SE2(64)
#undef ANNC_SE2
  }
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

}  // namespace

int launch_sparse_embedding2(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                             const void* ids, int ids_is_64, int64_t n, int64_t fallback,
                             float* out) {
  const int64_t total = n * dim;
  if (total == 0) return ANNC_OK;
  auto aligned16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  if (dim % 4 == 0 && aligned16(table) && aligned16(out) && n < (int64_t(1) << 40)) {
    return ids_is_64 ? launch_se2_vec(s, table, rows, dim, static_cast<const int64_t*>(ids), n,
                                      fallback, out)
                     : launch_se2_vec(s, table, rows, dim, static_cast<const int32_t*>(ids), n,
                                      fallback, out);
  }
  dim3 grid((unsigned)ceil_div(total, kThreads));
  if (ids_is_64)
    hipLaunchKernelGGL(sparse_embedding2_kernel<int64_t>, grid, dim3(kThreads), 0, s, table, rows,
                       dim, static_cast<const int64_t*>(ids), n, fallback, out);
  else
    hipLaunchKernelGGL(sparse_embedding2_kernel<int32_t>, grid, dim3(kThreads), 0, s, table, rows,
                       dim, static_cast<const int32_t*>(ids), n, fallback, out);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

// __reduce_mean (reduce_rewriter.cc:31-46): out[i] = (sum of |x| over the
// i-th run of m consecutive values) / m, one wave per output.  The lanes
// take strided values and a butterfly of lane shuffles adds their sums (the
// reference's cblas_sasum fixes no order either).
__global__ __launch_bounds__(kThreads) void abs_mean_kernel(const float* __restrict__ x, int64_t m,
                                                            int64_t n, float* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const float* __restrict__ row = x + i * m;
  float acc = 0.0f;
  for (int64_t j = lane; j < m; j += 64) acc += fabsf(row[j]);
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) out[i] = acc / static_cast<float>(static_cast<int>(m));
}

int launch_pooling(hipStream_t s, const int64_t* ids, const float* gathered, int64_t m, int64_t k,
                   int64_t n, const int64_t* ss, const int64_t* sl, float* out) {
  if (m * n == 0) return ANNC_OK;
  const bool aligned = ((reinterpret_cast<uintptr_t>(gathered) | reinterpret_cast<uintptr_t>(out)) &
                        15) == 0;
  if (n % 4 == 0 && aligned && m * k * n * 4 < (int64_t(1) << 31) && k < (int64_t(1) << 24)) {
    const int g = vec_group(n / 4);
    const dim3 grid((unsigned)ceil_div(m * g, kThreads));
    // rows of up to 48 positions: the one-round kernel, R = k rounded up to 16
    const int r = k == 0 ? 0 : k <= 16 ? 16 : k <= 32 ? 32 : k <= 48 ? 48 : 0;
    switch (g) {
#define ANNC_POOL_R(G, R)                                                                       \
  hipLaunchKernelGGL((pooling_round_kernel<G, R>), grid, dim3(kThreads), 0, s, ids, gathered, m, \
                     k, n, ss[0], ss[1], ss[2], sl[0], sl[1], sl[2], out)
#define ANNC_POOL(G)                                                                          \
  case G:                                                                                     \
    if (r == 16)                                                                              \
      ANNC_POOL_R(G, 16);                                                                     \
    else if (r == 32)                                                                         \
      ANNC_POOL_R(G, 32);                                                                     \
    else if (r == 48)                                                                         \
      ANNC_POOL_R(G, 48);                                                                     \
    else                                                                                      \
      hipLaunchKernelGGL(pooling_vec_kernel<G>, grid, dim3(kThreads), 0, s, ids, gathered, m, \
                         k, n, ss[0], ss[1], ss[2], sl[0], sl[1], sl[2], out);                \
    break;
      ANNC_POOL(1) ANNC_POOL(2) ANNC_POOL(4) ANNC_POOL(8) ANNC_POOL(16) ANNC_POOL(32) ANNC_POOL(64)
#undef ANNC_POOL
#undef ANNC_POOL_R
    }
    ANNC_HIP_TRY(hipGetLastError());
    return ANNC_OK;
  }
  hipLaunchKernelGGL(pooling_kernel, dim3((unsigned)ceil_div(m * n, kThreads)), dim3(kThreads), 0,
                     s, ids, gathered, m, k, n, ss[0], ss[1], ss[2], sl[0], sl[1], sl[2], out);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

int launch_abs_mean(hipStream_t s, const float* x, int64_t m, int64_t n, float* out) {
  if (n <= 0) return ANNC_OK;
  hipLaunchKernelGGL(abs_mean_kernel, dim3((unsigned)ceil_div(n * 64, kThreads)), dim3(kThreads),
                     0, s, x, m, n, out);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

int widen_i32(hipStream_t s, const int32_t* src, int64_t n, int64_t* dst) {
  if (n <= 0) return ANNC_OK;
  hipLaunchKernelGGL(widen_i32_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0, s,
                     src, n, dst);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

size_t nonzero_scan_temp_bytes(int64_t count) { return scan_temp_bytes(count); }

int nonzero_compact(hipStream_t s, const float* dense, int64_t count, int64_t dim,
                    const int64_t* seg_of_row, int one_d, int32_t* flags, int32_t* incl, void* tmp,
                    size_t tmp_bytes, int64_t cap, int32_t* out_idx, float* out_val) {
  ANNC_REQUIRE(count < (int64_t(1) << 31), "too many reduced values");
  if (count <= 0) return ANNC_OK;
  const dim3 grid((unsigned)ceil_div(count, kThreads));
  hipLaunchKernelGGL(nz_flag_kernel, grid, dim3(kThreads), 0, s, dense, count, flags);
  ANNC_HIP_TRY(hipGetLastError());
  ANNC_REQUIRE(tmp_bytes >= scan_temp_bytes(count), "scan scratch too small");
  const int rc = inclusive_sum(s, flags, incl, count, tmp);
  if (rc != ANNC_OK) return rc;
  if (out_idx) return nonzero_write(s, dense, count, dim, seg_of_row, one_d, flags, incl, cap,
                                    out_idx, out_val);
  return ANNC_OK;
}

int nonzero_write(hipStream_t s, const float* dense, int64_t count, int64_t dim,
                  const int64_t* seg_of_row, int one_d, const int32_t* flags, const int32_t* incl,
                  int64_t cap, int32_t* out_idx, float* out_val) {
  if (count <= 0 || cap <= 0) return ANNC_OK;
  const dim3 grid((unsigned)ceil_div(count, kThreads));
  hipLaunchKernelGGL(nz_write_kernel, grid, dim3(kThreads), 0, s, dense, count, dim, seg_of_row,
                     one_d, flags, incl, cap, out_idx, out_val);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

}  // namespace annc

// ---------------------------------------------------------------------------
// Device scratch of the allocation-free segment reduction
// (annc_hip_segment_reduce_noalloc): one copy per GPU, held until the process
// ends.  The first kNoAllocStatusBytes hold the status word kernels write
// when the caller passes none; the rest is the workspace.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr size_t kNoAllocStatusBytes = 256;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace annc {
namespace {
std::mutex g_scratch_mu;
std::map<int, char*> g_scratch_ptr;  // device -> address of that device's copy

// Address of `scratch` on the current device (looked up once per device;
// the host-side name is not a device address).
int noalloc_scratch(char** out) {
  int dev = 0;
  ANNC_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    char* ptr = nullptr;
    ANNC_HIP_TRY(hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch)));
    it = g_scratch_ptr.emplace(dev, ptr).first;
  }
  *out = it->second;
  return ANNC_OK;
}
}  // namespace
}  // namespace annc

extern "C" {

int annc_hip_embedding_bag(void* stream, const float* table, int64_t rows, int64_t dim,
                           const void* ids, int ids_is_64, const int64_t* offsets,
                           int64_t num_bags, int combiner, float* out, int64_t ldo) {
  using namespace annc;
  ANNC_REQUIRE(rows >= 0 && dim >= 1 && num_bags >= 0, "bad table or bag dimensions");
  ANNC_REQUIRE(ldo >= dim, "ldo < dim");
  ANNC_REQUIRE(combiner == ANNC_COMBINER_SUM || combiner == ANNC_COMBINER_MEAN,
               "combiner must be 0 or 1");
  if (num_bags == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(table && ids && offsets && out, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* status = stream_status(s);
  if (!status) return set_error(ANNC_RESOURCE_EXHAUSTED, "status allocation failed");
  BagArgs a{};
  a.table = table;
  a.rows = rows;
  a.dim = dim;
  a.ids = ids;
  a.ids_is_64 = ids_is_64;
  a.offsets = offsets;
  a.perm = nullptr;
  a.num_bags = num_bags;
  a.combiner = combiner;
  a.out = out;
  a.ldo = ldo;
  a.status = status;
  int rc = launch_bag(a, s);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

int annc_hip_segment_reduce(void* stream, const float* data, int64_t rows, int64_t dim,
                            const void* indices, int indices_is_64, const int64_t* seg_ids,
                            int64_t seg_stride, int64_t n, int combiner, int64_t batch,
                            float* out, int seg_sorted) {
  using namespace annc;
  ANNC_REQUIRE(rows >= 0 && dim >= 1 && n >= 0 && batch >= 0 && seg_stride >= 1,
               "bad dimensions");
  ANNC_REQUIRE(combiner == ANNC_COMBINER_SUM || combiner == ANNC_COMBINER_MEAN,
               "combiner must be 0 or 1");
  if (batch == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(data && out && (n == 0 || (indices && seg_ids)), "null pointer");
  ANNC_REQUIRE(seg_sorted == 0 || seg_sorted == 1, "seg_sorted must be 0 or 1");
  int rc = segment_reduce(static_cast<hipStream_t>(stream), data, rows, dim, indices,
                          indices_is_64, seg_ids, seg_stride, n, combiner, batch, out, seg_sorted);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

int annc_hip_segment_reduce_noalloc(void* stream, const float* data, int64_t rows, int64_t dim,
                                    const void* indices, int indices_is_64,
                                    const int64_t* seg_ids, int64_t seg_stride, int64_t n,
                                    int combiner, int64_t batch, float* out, int seg_sorted,
                                    int32_t* status) {
  using namespace annc;
  ANNC_REQUIRE(rows >= 0 && dim >= 1 && n >= 0 && batch >= 0 && seg_stride >= 1,
               "bad dimensions");
  ANNC_REQUIRE(combiner == ANNC_COMBINER_SUM || combiner == ANNC_COMBINER_MEAN,
               "combiner must be 0 or 1");
  if (batch == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(data && out && (n == 0 || (indices && seg_ids)), "null pointer");
  ANNC_REQUIRE(seg_sorted == 0 || seg_sorted == 1, "seg_sorted must be 0 or 1");
  hipStream_t s = static_cast<hipStream_t>(stream);
  SegPlan plan;
  int rc = segment_reduce_plan(n, batch, seg_sorted, s, &plan);
  if (rc != ANNC_OK) return rc;
  constexpr size_t kMax = kNoAllocScratchBytes - kNoAllocStatusBytes;
  ANNC_REQUIRE(plan.bytes <= kMax,
               "segment reduction of %lld positions into %lld segments needs %zu bytes of "
               "workspace, above the %zu bytes of the allocation-free entry's scratch",
               (long long)n, (long long)batch, plan.bytes, kMax);
  char* base = nullptr;
  rc = noalloc_scratch(&base);
  if (rc != ANNC_OK) return rc;
  int* st = status ? reinterpret_cast<int*>(status) : reinterpret_cast<int*>(base);
  rc = segment_reduce_run(s, data, rows, dim, indices, indices_is_64, seg_ids, seg_stride, n,
                          combiner, batch, out, plan, base + kNoAllocStatusBytes, st);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

int annc_hip_sparse_embedding2(void* stream, const float* table, int64_t rows, int64_t dim,
                               const void* ids, int ids_is_64, int64_t n, int64_t fallback_row,
                               float* out) {
  using namespace annc;
  ANNC_REQUIRE(rows >= 1 && dim >= 1 && n >= 0, "bad dimensions");
  ANNC_REQUIRE(fallback_row >= 0 && fallback_row < rows, "fallback row out of range");
  if (n == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(table && ids && out, "null pointer");
  int rc = launch_sparse_embedding2(static_cast<hipStream_t>(stream), table, rows, dim, ids,
                                    ids_is_64, n, fallback_row, out);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

int annc_hip_pooling(void* stream, const int64_t* ids, const float* gathered, int64_t m,
                     int64_t k, int64_t n, const int64_t* slice_starts3,
                     const int64_t* slice_limits3, float* out) {
  using namespace annc;
  ANNC_REQUIRE(m >= 0 && k >= 0 && n >= 0, "bad dimensions");
  ANNC_REQUIRE(slice_starts3 && slice_limits3, "null slice bounds");
  if (m * n == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(ids && gathered && out, "null pointer");
  int rc = launch_pooling(static_cast<hipStream_t>(stream), ids, gathered, m, k, n, slice_starts3,
                          slice_limits3, out);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

}  // extern "C"
