// gemm.hip -- fp32 GEMM on CDNA4 matrix cores (gfx950).
//
// Engine behind the XLA custom calls __matmul, __matmul_add,
// __matmul_add_relu, __batch_matmul and __layout_matmul
// (annc/service/cpu/gemm_rewriter.cc:136-281), which the reference runs as
// OpenBLAS / kpgemm sgemm calls followed by scalar epilogue loops.
//
// Design (one 256-thread workgroup = 4 wave64 per output tile):
//   * v_mfma_f32_32x32x2f32: each wave owns BLK_M x BLK_N 32x32 accumulator
//     blocks (16 fp32 per lane each).
//   * A tiles [BM x 32] are staged through LDS, double buffered, rows padded
//     to 36 floats so the 16-byte fragment reads are bank-conflict free.
//     Each lane half h (lanes 0-31 / 32-63) consumes k = 16h .. 16h+15 of a
//     32-wide k block, so one ds_read_b128 feeds 4 MFMA steps.
//   * Row-major B tiles [32 x BN] are staged through LDS (double buffered)
//     and read one float per lane per step.  layout_matmul-packed B skips
//     LDS: each wave loads its fragments straight from global memory, one
//     coalesced 16-byte load per lane per 4 steps, prefetched a block ahead.
//   * Epilogue fuses the addend matrix (__matmul_add*), a bias vector,
//     ReLU (std::max(x, 0.f) semantics) or sigmoid before the single store.
//   * Tiles are numbered so that each XCD (workgroup id mod 8) receives a
//     contiguous run of tiles sharing A rows, keeping them in its own L2.
//   * The packed pipeline also has a v_mfma_f32_16x16x4f32 form (16x16
//     blocks), selected only by the ANNC_GEMM_PIPE tuning variable.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.h"
#include "layout_pack.h"

namespace annc {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;          // k block
constexpr int kALd = kBK + 4;    // padded LDS row of the A tile (floats)
constexpr int kThreads = 256;

struct GemmParams {
  const float* a;
  const float* b;
  const float* e;
  const float* bias;
  float* c;
  int64_t lda, ldb, lde, ldc;
  int64_t stride_a, stride_b, stride_e, stride_c;
  int m, n, k;
  int tiles_m, tiles_n;
  int epilogue;
  int a_vec;  // A rows can be read as aligned float4
  int b_vec;  // row-major B rows can be read as aligned float4
  int b_dense;  // B is a dense row-major [K, N] block (ldb == N), 16-byte aligned
  // small kernel with K split over gridDim.y workgroups: each writes its
  // partial sums (no epilogue) to part[split][batch][M][N]
  float* part;
};

__device__ __forceinline__ float apply_epilogue(float v, int epilogue) {
  if (epilogue & ANNC_EPI_RELU) v = (v < 0.0f) ? 0.0f : v;
  if (epilogue & ANNC_EPI_SIGMOID) v = 1.0f / (1.0f + expf(-v));
  return v;
}

template <int WAVES_M, int WAVES_N, int BLK_M, int BLK_N, bool PACKED>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmParams p) {
  constexpr int BM = WAVES_M * BLK_M * 32;
  constexpr int BN = WAVES_N * BLK_N * 32;
  constexpr int A_CHUNKS = BM * kBK / 4 / kThreads;  // float4 per thread per A block
  constexpr int B_CHUNKS = kBK * BN / 4 / kThreads;  // float4 per thread per B block
  static_assert(WAVES_M * WAVES_N * 64 == kThreads, "4 waves per workgroup");
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small");

  __shared__ __attribute__((aligned(16))) float As[2][BM * kALd];
  __shared__ __attribute__((aligned(16))) float Bs[PACKED ? 1 : 2][PACKED ? 4 : kBK * BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int half = lane >> 5;   // which 16-wide k half this lane feeds
  const int l32 = lane & 31;

  // XCD-aware tile order: workgroup i runs on XCD i % 8.
  int tile = blockIdx.x;
  const int T = p.tiles_m * p.tiles_n;
  if ((T & 7) == 0) tile = (tile & 7) * (T >> 3) + (tile >> 3);
  const int m0 = (tile / p.tiles_n) * BM;
  const int n0 = (tile % p.tiles_n) * BN;

  const int64_t z = blockIdx.z;
  const float* __restrict__ A = p.a + z * p.stride_a;
  const float* __restrict__ B = p.b + z * p.stride_b;
  const int M = p.m, N = p.n, K = p.k;
  const int KT = (K + kBK - 1) / kBK;

  // ---- global -> register loaders ----
  f32x4 a_reg[A_CHUNKS];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int c = 0; c < A_CHUNKS; ++c) {
      const int lin = tid + kThreads * c;
      const int row = lin >> 3;
      const int col = (lin & 7) * 4;
      const int gm = m0 + row;
      const int gk = kt * kBK + col;
      if (gm < M && p.a_vec && gk + 3 < K) {
        a_reg[c] = *reinterpret_cast<const f32x4*>(A + (int64_t)gm * p.lda + gk);
      } else {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (gm < M && gk + e < K) ? A[(int64_t)gm * p.lda + gk + e] : 0.0f;
        a_reg[c] = v;
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int c = 0; c < A_CHUNKS; ++c) {
      const int lin = tid + kThreads * c;
      const int row = lin >> 3;
      const int col = (lin & 7) * 4;
      *reinterpret_cast<f32x4*>(&As[buf][row * kALd + col]) = a_reg[c];
    }
  };

  f32x4 b_reg[PACKED ? 1 : B_CHUNKS];
  auto load_b = [&](int kt) {
#pragma unroll
    for (int c = 0; c < B_CHUNKS; ++c) {
      const int lin = tid + kThreads * c;
      const int row = lin / (BN / 4);
      const int col = (lin % (BN / 4)) * 4;
      const int gk = kt * kBK + row;
      const int gn = n0 + col;
      if (gk < K && p.b_vec && gn + 3 < N) {
        b_reg[c] = *reinterpret_cast<const f32x4*>(B + (int64_t)gk * p.ldb + gn);
      } else {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (gk < K && gn + e < N) ? B[(int64_t)gk * p.ldb + gn + e] : 0.0f;
        b_reg[c] = v;
      }
    }
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int c = 0; c < B_CHUNKS; ++c) {
      const int lin = tid + kThreads * c;
      const int row = lin / (BN / 4);
      const int col = (lin % (BN / 4)) * 4;
      *reinterpret_cast<f32x4*>(&Bs[buf][row * BN + col]) = b_reg[c];
    }
  };

  // Packed B: fragments straight from global memory.
  const int kf = K & ~31;
  const int nf = N & ~31;
  f32x4 bp_cur[PACKED ? BLK_N : 1][4];
  f32x4 bp_nxt[PACKED ? BLK_N : 1][4];
  auto load_bp = [&](int kt, f32x4 (&dst)[PACKED ? BLK_N : 1][4]) {
#pragma unroll
    for (int bn = 0; bn < (PACKED ? BLK_N : 1); ++bn) {
      const int pn = (n0 >> 5) + wn * BLK_N + bn;
      const bool full = (kt * kBK + kBK <= kf) && ((pn + 1) * 32 <= nf);
      if (full) {
        const f32x4* src = reinterpret_cast<const f32x4*>(
            B + ((int64_t)pn * (kf >> 5) + kt) * 1024 + lane * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[bn][q] = src[q * 64];
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int gk = kt * kBK + 16 * half + 4 * q + e;
            const int gn = pn * 32 + l32;
            v[e] = (gk < K && gn < N) ? B[layout_pack_offset(gk, gn, K, N)] : 0.0f;
          }
          dst[bn][q] = v;
        }
      }
    }
  };

  f32x16 acc[BLK_M][BLK_N];
#pragma unroll
  for (int i = 0; i < BLK_M; ++i)
#pragma unroll
    for (int j = 0; j < BLK_N; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 af[BLK_M];
      f32x4 bf[BLK_N];
#pragma unroll
      for (int i = 0; i < BLK_M; ++i) {
        const int row = wm * BLK_M * 32 + i * 32 + l32;
        af[i] = *reinterpret_cast<const f32x4*>(&As[buf][row * kALd + 16 * half + 4 * q]);
      }
#pragma unroll
      for (int j = 0; j < BLK_N; ++j) {
        if constexpr (PACKED) {
          bf[j] = bp_cur[j][q];
        } else {
          const int col = wn * BLK_N * 32 + j * 32 + l32;
#pragma unroll
          for (int e = 0; e < 4; ++e) bf[j][e] = Bs[buf][(16 * half + 4 * q + e) * BN + col];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < BLK_M; ++i)
#pragma unroll
          for (int j = 0; j < BLK_N; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][e], bf[j][e], acc[i][j], 0, 0, 0);
    }
  };

  // ---- main loop: one barrier per k block ----
  load_a(0);
  if constexpr (PACKED) load_bp(0, bp_cur); else load_b(0);
  store_a(0);
  if constexpr (!PACKED) store_b(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      load_a(kt + 1);
      if constexpr (PACKED) load_bp(kt + 1, bp_nxt); else load_b(kt + 1);
    }
    compute(cur);
    if (more) {
      store_a(cur ^ 1);
      if constexpr (PACKED) {
#pragma unroll
        for (int j = 0; j < BLK_N; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) bp_cur[j][q] = bp_nxt[j][q];
      } else {
        store_b(cur ^ 1);
      }
    }
    __syncthreads();
  }

  // ---- fused epilogue ----
  const float* __restrict__ E = p.e ? p.e + z * p.stride_e : nullptr;
  float* __restrict__ C = p.c + z * p.stride_c;
#pragma unroll
  for (int i = 0; i < BLK_M; ++i) {
#pragma unroll
    for (int j = 0; j < BLK_N; ++j) {
      const int col = n0 + wn * BLK_N * 32 + j * 32 + l32;
      if (col >= N) continue;
      const float bias = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * BLK_M * 32 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (E) v += E[(int64_t)row * p.lde + col];
        if (p.bias) v += bias;
        C[(int64_t)row * p.ldc + col] = apply_epilogue(v, p.epilogue);
      }
    }
  }
}

// Skinny-N path, N <= 4 (a tower's scoring layer); for N < 32 the packed
// layout is row-major, so packed and plain B share it.  16 lanes per row,
// 4 rows per wave.  Lane
// t of a row multiplies A[row, 64i + 4t .. 64i + 4t + 3] (one float4 per
// chunk i) with the matching B rows, and the 16 partial sums are combined with
// DPP row rotations, after which every lane of the row holds its sums.  Rows
// past M are clamped to M - 1 so every lane takes part in the DPP; only the
// store is predicated.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int N>
__global__ __launch_bounds__(kThreads) void gemv_rows_kernel(GemmParams p) {
  constexpr int kRowLanes = 16;
  const int t = threadIdx.x & (kRowLanes - 1);
  const int64_t row = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / kRowLanes;
  const int64_t z = blockIdx.z;
  const int64_t r = row < p.m ? row : (int64_t)p.m - 1;
  const float* __restrict__ A = p.a + z * p.stride_a + r * p.lda;
  const float* __restrict__ B = p.b + z * p.stride_b;
  const int K = p.k;
  float part[N];
#pragma unroll
  for (int j = 0; j < N; ++j) part[j] = 0.0f;
  int kk = 4 * t;
  if (p.a_vec && p.b_dense) {
    // B rows kk .. kk+3 are the 4N floats at B + kk*N: element (e, j) is e*N + j
    auto chunk = [&](const f32x4& av, const f32x4* bv) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < N; ++j) part[j] += av[e] * bv[(e * N + j) >> 2][(e * N + j) & 3];
    };
    for (; kk + 195 < K; kk += 256) {  // four chunks in flight per lane
      f32x4 av[4], bv[4][N];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        av[u] = *reinterpret_cast<const f32x4*>(A + kk + 64 * u);
#pragma unroll
        for (int c = 0; c < N; ++c)
          bv[u][c] = *reinterpret_cast<const f32x4*>(B + (int64_t)(kk + 64 * u) * N + 4 * c);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) chunk(av[u], bv[u]);
    }
    for (; kk + 3 < K; kk += 64) {
      f32x4 bv[N];
      const f32x4 av = *reinterpret_cast<const f32x4*>(A + kk);
#pragma unroll
      for (int c = 0; c < N; ++c) bv[c] = *reinterpret_cast<const f32x4*>(B + (int64_t)kk * N + 4 * c);
      chunk(av, bv);
    }
  }
  // other layouts (B rows not dense or not aligned, A rows not aligned):
  // scalar loads in the same k order, four chunks in flight per lane
  for (; kk + 195 < K; kk += 256) {
    float av[4][4], bv[4][4][N];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = kk + 64 * u + e;
        av[u][e] = A[k];
#pragma unroll
        for (int j = 0; j < N; ++j) bv[u][e][j] = B[(int64_t)k * p.ldb + j];
      }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < N; ++j) part[j] += av[u][e] * bv[u][e][j];
  }
  for (; kk < K; kk += 64) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (kk + e < K) {
        const float av = A[kk + e];
#pragma unroll
        for (int j = 0; j < N; ++j) part[j] += av * B[(int64_t)(kk + e) * p.ldb + j];
      }
    }
  }
  float v = 0.0f;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float s = part[j];
    s = dpp_add<0x128>(s);  // row_ror:8
    s = dpp_add<0x124>(s);  // row_ror:4
    s = dpp_add<0x04E>(s);  // quad_perm [2,3,0,1]
    s = dpp_add<0x0B1>(s);  // quad_perm [1,0,3,2]
    if (t == j) v = s;
  }
  if (row < p.m && t < N) {
    if (p.e) v += p.e[z * p.stride_e + row * p.lde + t];
    if (p.bias) v += p.bias[t];
    p.c[z * p.stride_c + row * p.ldc + t] = apply_epilogue(v, p.epilogue);
  }
}

// Small row-major GEMMs (few output tiles, e.g. the 512x256x256 custom call):
// one 32x32 output block per workgroup and the K dimension split over its W
// waves (wave w takes k-blocks w, w+W, ...), so a 512x256 output still runs
// 128 workgroups x W waves.  Each wave loads its MFMA operands straight from
// global memory -- A as one float4 per lane per 4 k (row l32, k chunk
// 16*half + 4q), B as one float per lane per k (row k, column l32) -- one
// k-block ahead of the MFMAs, with two accumulator chains.  Full k-blocks
// load unguarded (rows and columns past the edge are clamped, computed and
// never stored), so the loads carry no branches; the K % 32 tail is one
// guarded block afterwards.  The W partial blocks meet in LDS and wave v
// adds registers 4v..4v+3 over w = 0..W-1 in that order before the fused
// epilogue.
template <int W, bool AVEC, bool PACKED = false, bool KSPLIT = false>
__global__ __launch_bounds__(64 * W) void gemm_small_kernel(GemmParams p) {
  static_assert(W == 4 || W == 8, "4 or 8 waves");
  // PACKED: B in the layout_matmul format: a k-block of the workgroup's
  // full 32-column panel is 1 KiB whose quad q holds, at float4 `lane`, this
  // lane's B operand of MFMA steps 4q..4q+3 -- the same values, in the same
  // order, as the row-major loads.  The partial last panel of N % 32 != 0
  // (tpan) reads the format's row-major [K, N % 32] N-tail region as
  // row-major B.
  __shared__ float red[W][16][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const int m0 = (blockIdx.x / p.tiles_n) * 32;
  const int n0 = (blockIdx.x % p.tiles_n) * 32;
  const int64_t z = blockIdx.z;
  const int M = p.m, N = p.n, K = p.k;
  const int KF = K >> 5;  // full k-blocks
  // this workgroup's k-blocks [kb0, kb1) (all of them without a K split);
  // the K % 32 tail goes to the last split
  const int split = KSPLIT ? (int)blockIdx.y : 0, splits = KSPLIT ? (int)gridDim.y : 1;
  const int kb0 = KSPLIT ? KF * split / splits : 0;
  const int kb1 = KSPLIT ? KF * (split + 1) / splits : KF;
  const bool last_split = !KSPLIT || split == splits - 1;
  const int col = n0 + l32;
  const bool col_ok = col < N;
  const float* __restrict__ arow = p.a + z * p.stride_a + (int64_t)min(m0 + l32, M - 1) * p.lda;
  const int nf = N & ~31;
  const bool tpan = PACKED && n0 >= nf;  // the partial panel (wave-uniform)
  const int nt = N - nf;
  const float* __restrict__ bcol =
      tpan ? p.b + z * p.stride_b + (int64_t)nf * K + min(col - nf, nt - 1)
           : p.b + z * p.stride_b + min(col, N - 1);
  const int64_t ldb = tpan ? nt : p.ldb;
  // PACKED: this lane's float4 in the panel's k-block 0, and the row-major
  // K-tail rows [K - 32*KF, nf] of the full panels that follow the blocks
  const float* __restrict__ bpan = p.b + z * p.stride_b + (int64_t)(n0 >> 5) * KF * 1024 + 4 * lane;
  const float* __restrict__ btail = p.b + z * p.stride_b + (int64_t)nf * KF * 32 + min(col, nf - 1);
  // the addend of the four output registers this wave finishes (wave & 3),
  // fetched before the k-loop; without an addend the loads re-read C and are
  // ignored, so no wave branches around them
  const float* __restrict__ E = p.e ? p.e + z * p.stride_e : nullptr;
  float* __restrict__ C = p.c + z * p.stride_c;
  const float* __restrict__ esrc = E ? E : C;
  const int64_t lde = E ? p.lde : p.ldc;
  float e_pre[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int orow = min(m0 + 8 * (wave & 3) + 4 * half + i, M - 1);
    e_pre[i] = esrc[(int64_t)orow * lde + min(col, N - 1)];
  }

  f32x4 af[2][4];
  float bf[2][16];
  auto load = [&](int kt, int buf) {
    const int kb = kt * 32 + 16 * half;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (AVEC) {
        af[buf][q] = *reinterpret_cast<const f32x4*>(arow + kb + 4 * q);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) af[buf][q][e] = arow[kb + 4 * q + e];
      }
      if (PACKED && !tpan) {
        const f32x4 bq = *reinterpret_cast<const f32x4*>(bpan + (int64_t)kt * 1024 + 256 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) bf[buf][4 * q + e] = bq[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) bf[buf][4 * q + e] = bcol[(int64_t)(kb + 4 * q + e) * ldb];
      }
    }
  };
  f32x16 acc[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  auto mma = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc[e & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[buf][q][e], bf[buf][4 * q + e],
                                                          acc[e & 1], 0, 0, 0);
  };
  if (kb0 + wave < kb1) {
    // blocks kb0+wave, kb0+wave+W, ...; the prefetch of a block past the
    // end re-reads the current one instead of branching
    // sched_barrier keeps each prefetch issued ahead of the MFMAs it overlaps
    load(kb0 + wave, 0);
    for (int kt = kb0 + wave; kt < kb1; kt += 2 * W) {
      load(kt + W < kb1 ? kt + W : kt, 1);
      __builtin_amdgcn_sched_barrier(0);
      mma(0);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + W >= kb1) break;
      load(kt + 2 * W < kb1 ? kt + 2 * W : kt + W, 0);
      __builtin_amdgcn_sched_barrier(0);
      mma(1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if ((K & 31) && last_split && wave == (KF - kb0) % W) {
    const int kb = KF * 32 + 16 * half;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = kb + 4 * q + e;
        af[0][q][e] = k < K ? arow[k] : 0.0f;
        if (PACKED && !tpan)
          bf[0][4 * q + e] = k < K ? btail[(int64_t)(k - KF * 32) * nf] : 0.0f;
        else
          bf[0][4 * q + e] = k < K ? bcol[(int64_t)k * ldb] : 0.0f;
      }
    mma(0);
  }
  acc[0] += acc[1];
#pragma unroll
  for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[0][r];
  __syncthreads();
  if (wave >= 4) return;
  const float bias = (p.bias && col_ok) ? p.bias[col] : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * wave + i;
    float v = red[0][r][lane];
#pragma unroll
    for (int w = 1; w < W; ++w) v += red[w][r][lane];
    const int orow = m0 + 8 * wave + 4 * half + i;  // 8*(r>>2) + 4*half + (r&3)
    if (orow >= M || !col_ok) continue;
    if constexpr (KSPLIT) {
      p.part[(((int64_t)split * gridDim.z + z) * M + orow) * N + col] = v;
      continue;
    }
    if (E) v += e_pre[i];
    if (p.bias) v += bias;
    C[(int64_t)orow * p.ldc + col] = apply_epilogue(v, p.epilogue);
  }
}

// The K-split small GEMM's second launch: each output is its splits' partial
// sums added in split order, then the addend, the bias and the epilogue, as
// the one-launch form adds them to its wave sum.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p, int splits,
                                                            int64_t batch) {
  const int64_t total = batch * p.m * p.n;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t z = i / ((int64_t)p.m * p.n);
  const int64_t rem = i % ((int64_t)p.m * p.n);
  const int64_t row = rem / p.n, col = rem % p.n;
  float v = p.part[i];
  for (int s = 1; s < splits; ++s) v += p.part[(int64_t)s * total + i];
  if (p.e) v += p.e[z * p.stride_e + row * p.lde + col];
  if (p.bias) v += p.bias[col];
  p.c[z * p.stride_c + row * p.ldc + col] = apply_epilogue(v, p.epilogue);
}

// ---------------------------------------------------------------------------
// Packed-B pipelined kernel (the __layout_matmul path; row-major B with BRM;
// a partial last 32-column panel with NTAIL).
//
// Operand tiles stream global -> LDS through gfx950's 16-byte LDS-DMA loads
// (global_load_lds_dwordx4: lane i of a wave writes bytes [16i, 16i+16) of a
// 1 KiB LDS block), S stages deep, so no VGPRs stage the data and up to S-2
// stages are in flight while the MFMAs run on the oldest.  A stage holds
// one 32-k block.  One barrier per stage, halfway through it:
// a wave waits for its own DMAs of the next stage (vmcnt), the barrier
// publishes everyone's, and the slot of the previous stage is refilled.  The
// next stage's first fragments are then read under the current stage's last
// MFMAs, so the stage boundary itself has no barrier or LDS-latency gap.
//   * WM x WN waves own BLK_M x BLK_N 32x32 accumulator blocks each; with
//     KS = 2 a second group of WM x WN waves takes the other half of every
//     k-block (quads 2-3) and the two partial tiles are added through LDS
//     before the epilogue.  NACC = 2 alternates two accumulator chains per
//     block so a wave always has an independent MFMA to issue.
//   * A block = 8 full rows x 32 k (eight 128-byte lines per instruction);
//     lane i loads row i/8, 16-byte chunk (i%8) ^ swz(row), so each MFMA
//     fragment read (row = lane%32, chunk 4*(lane/32)+q) hits 64 distinct
//     banks: swz(row) = (row & 7) ^ ((row >> 3) & 1).
//   * B block = 1 KiB of the packed panel, already in MFMA-fragment order.
//     With BRM the kernel reads row-major B (rows 16-byte aligned) instead:
//     a B block is eight 128-byte row segments of one 32-column panel, rows
//     k and k+16 of the stage side by side, and a fragment is four 4-byte
//     LDS reads (the packed block's k order, so both forms give the same
//     bits); no packing pass runs.
//   * The DMAs are inline asm so the compiler neither tracks them nor adds
//     its conservative vmcnt(0) before LDS reads; the kernel counts them
//     itself (wait_vmcnt) and fences the barrier as asm as well.
//   * Rows past M and panels past N are clamped for loading and never
//     stored; a K tail (K % 32) is folded in after the loop from the
//     packed format's row-major tail regions with guarded loads.
//   * NTAIL: the partial panel's B blocks load with four 4-byte DMAs each
//     (the packed format's N-tail region, or the row-major rows), columns
//     clamped to N - 1.
// ---------------------------------------------------------------------------
namespace pipe {

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 16 bytes per lane from `src` into LDS at `lds_base + 16*lane`; lds_base is
// wave-uniform.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory");
}

// 4 bytes per lane from `src` into LDS at `lds_base + 4*lane` (rows that
// are not 16-byte aligned).
__device__ __forceinline__ void dma4(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Barrier with no LDS wait: for points where this wave's LDS reads of the
// slot about to be refilled were consumed by MFMAs long before.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ int a_swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }

}  // namespace pipe

template <int WM, int WN, int BLK_M, int BLK_N, int S, int NACC, int KS, bool A16, bool BRM,
          bool ZMAP, bool MI16 = false, bool NTAIL = false>
__global__ __launch_bounds__(64 * WM * WN * KS) void gemm_packed_pipe_kernel(GemmParams p) {
  static_assert(NACC == 1 || NACC == 2, "one or two accumulator chains");
  static_assert(KS == 1 || KS == 2, "one or two k groups");
  // MI16: 16x16 accumulator blocks on v_mfma_f32_16x16x4f32 (one k group,
  // packed B, K % 32 == 0).  A fragment step covers 16 k: lane l feeds k =
  // 4*(l/16) + s at MFMA step s, so one 16-byte LDS read per operand block
  // serves the 4 steps, from the same A and packed-B stage layouts.
  static_assert(!MI16 || (KS == 1 && !BRM), "16x16 blocks: one k group, packed B");
  // NTAIL: N % 32 != 0.  The last, partial 32-column panel loads its B
  // blocks with four 4-byte DMAs each, from the packed format's N-tail
  // region (row-major [K, N % 32] after the full panels) or from the
  // row-major B rows, each lane's column clamped to N - 1 (columns past N
  // are computed and never stored).
  static_assert(!NTAIL || !MI16, "N tail: 32x32 blocks");
  constexpr int MB = MI16 ? 16 : 32;               // rows and columns of an MFMA block
  constexpr int NR = MI16 ? 4 : 16;                // accumulator registers per block
  using AccT = std::conditional_t<MI16, f32x4, f32x16>;
  constexpr int NT = WM * WN;                      // waves per k group
  constexpr int NW = NT * KS;
  constexpr int NQ = MI16 ? 2 : 4 / KS;            // fragment steps per wave per k-block
  constexpr int BM = WM * BLK_M * MB, BN = WN * BLK_N * MB;
  static_assert(BN % 32 == 0, "whole 32-column panels");
  constexpr int NA = BM / 8, NB = BN / 8, NBLK = NA + NB;  // 1 KiB blocks per stage
  static_assert(NBLK % NW == 0, "stage blocks split evenly over the waves");
  static_assert(S >= 3 && S <= 4, "3 or 4 stages: the next stage is published mid-stage");
  static_assert(KS == 1 || NT * 2 * BLK_M * BLK_N * 2 <= S * NBLK, "exchange fits in LDS");
  constexpr int LPW = NBLK / NW;                    // 1 KiB blocks per wave per k-block
  // A rows that are not 16-byte aligned load each A block with four 4-byte
  // DMAs (two rows each); the first LPA blocks of every wave are A blocks.
  static_assert(A16 || NA % NW == 0, "A blocks split evenly over the waves");
  constexpr int LPA = NA / NW;
  constexpr int DMAS = A16 ? LPW : LPW + 3 * LPA;  // DMA instructions per wave per k-block
  constexpr uint32_t kStageBytes = NBLK * 1024;
  __shared__ __attribute__((aligned(1024))) f32x4 lds[S][NBLK * 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave / NT;                         // k group: quads kg*NQ .. kg*NQ+NQ-1
  const int wt = wave % NT;
  const int wm = wt / WN;
  const int wn = wt % WN;
  const int l32 = lane & 31;
  const int half = lane >> 5;

  // Workgroups are dealt to the 8 XCDs round-robin by linear id.  XCD c
  // takes the contiguous range c*total/8 .. (c+1)*total/8 - 1 of the tiles
  // (row-major tiles; with ZMAP, of the whole (batch, tile) space, tiles then
  // batches), so tiles that share A rows, B panels or a batch's operands
  // share that XCD's L2.  ZMAP is for batched launches only: the one-batch
  // form avoids its division by T.
  int tile = blockIdx.x;
  uint32_t zi = blockIdx.z;
  const int T = p.tiles_m * p.tiles_n;
  if constexpr (ZMAP) {
    const int total = T * (int)gridDim.z;
    if ((total & 7) == 0) {
      const int lin = (int)blockIdx.x + T * (int)blockIdx.z;
      const int lg = (lin & 7) * (total >> 3) + (lin >> 3);
      zi = (uint32_t)(lg / T);
      tile = lg % T;
    }
  } else {
    if ((T & 7) == 0) tile = (tile & 7) * (T >> 3) + (tile >> 3);
  }
  const int m0 = (tile / p.tiles_n) * BM;
  const int n0 = (tile % p.tiles_n) * BN;
  const int64_t z = zi;
  const float* __restrict__ A = p.a + z * p.stride_a;
  const float* __restrict__ B = p.b + z * p.stride_b;
  const int M = p.m, N = p.n, K = p.k;
  const int KT = K >> 5;          // full k-blocks
  const int KB = KT;              // stages
  const int panels = N >> 5;      // full 32-column panels
  const int npan = NTAIL ? (N + 31) >> 5 : panels;
  const int nt = N - 32 * panels;  // NTAIL: columns of the partial panel

  // bias of this lane's columns, fetched before the pipeline starts
  const int fl = MI16 ? (lane & 15) : l32;  // this lane's row / column in an MFMA block
  float bias_v[BLK_N];
#pragma unroll
  for (int j = 0; j < BLK_N; ++j) {
    const int col = n0 + (wn * BLK_N + j) * MB + fl;
    bias_v[j] = (p.bias && col < N) ? p.bias[col] : 0.0f;
  }

  // this wave's DMA sources (advanced by one k-block per stage) and LDS slots
  const float* src[LPW];
  std::conditional_t<BRM, int64_t, int> step[LPW];  // floats per k-block
  uint32_t dst[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int b = wave + NW * i;
    dst[i] = __builtin_amdgcn_readfirstlane(pipe::lds_offset(&lds[0][b * 64]));
    if (b < NA) {
      const int trow = b * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ pipe::a_swizzle(trow);
      const int row = min(m0 + trow, M - 1);
      src[i] = A + (int64_t)row * p.lda + chunk * 4;
      step[i] = 32;
    } else {
      const int bb = b - NA;
      const int pn = min((n0 >> 5) + (bb >> 2), npan - 1);
      if constexpr (BRM) {
        // Row-major B: block bb&3 of a panel's stage holds the 128-byte row
        // segments of LDS slots 8*(bb&3) .. +7, slot s holding k = s/2 +
        // 16*(s%2), so rows k and k+16 sit side by side
        const int slot = 8 * (bb & 3) + (lane >> 3);
        const int kr = (slot >> 1) + 16 * (slot & 1);
        src[i] = B + (int64_t)kr * p.ldb + pn * 32 + (lane & 7) * 4;
        step[i] = 32 * p.ldb;
      } else {
        src[i] = B + (int64_t)pn * KT * 1024 + (bb & 3) * 256 + lane * 4;
        step[i] = 1024;
      }
    }
  }
  // NTAIL: 4-byte DMA sources of the partial panel's B blocks.  Instruction
  // j of block i fills LDS floats [64j, 64j+64) of its 1 KiB block: lane l
  // writes float 64j + l.  Packed: that float is lane L = 16j + l/4, step
  // e = l%4 of quad q = bb&3, i.e. k = 16*(L/32) + 4q + e, n = L%32 of the
  // k-block.  Row-major: slot 8q + 2j + l/32 (row k = slot/2 + 16*(slot%2)),
  // column l%32.
  bool tpart[LPW];
  const float* tsrc[NTAIL ? LPW : 1][4];
  int64_t tstep = 0;
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int b = wave + NW * i;
    tpart[i] = false;
    if constexpr (NTAIL) {
      const int bb = b - NA;
      const int pn = min((n0 >> 5) + (bb >> 2), npan - 1);
      tpart[i] = b >= NA && pn == panels;
      const int q = bb & 3;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (BRM) {
          const int slot = 8 * q + 2 * j + (lane >> 5);
          const int kr = (slot >> 1) + 16 * (slot & 1);
          tsrc[i][j] = B + (int64_t)kr * p.ldb + min(32 * panels + (lane & 31), N - 1);
          tstep = 32 * p.ldb;
        } else {
          const int L = 16 * j + (lane >> 2);
          const int kk = 16 * (L >> 5) + 4 * q + (lane & 3);
          tsrc[i][j] = B + (int64_t)32 * panels * K + (int64_t)kk * nt + min(L & 31, nt - 1);
          tstep = (int64_t)32 * nt;
        }
      }
    }
  }
  // 4-byte DMA sources of the A blocks: instruction j of block i fills LDS
  // bytes [256j, 256j+256), i.e. rows 2j, 2j+1 of the block; lane l writes
  // word l%4 of 16-byte chunk (l%32)/4 of row 2j + l/32, which holds k chunk
  // ((l%32)/4) ^ swz(row) -- the same swizzled layout the 16-byte DMA writes.
  const float* src4[A16 ? 1 : LPA][4];
  if constexpr (!A16) {
#pragma unroll
    for (int i = 0; i < LPA; ++i) {
      const int b = wave + NW * i;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int trow = b * 8 + 2 * j + (lane >> 5);
        const int chunk = ((lane & 31) >> 2) ^ pipe::a_swizzle(trow);
        const int row = min(m0 + trow, M - 1);
        src4[i][j] = A + (int64_t)row * p.lda + chunk * 4 + (lane & 3);
      }
    }
  }
  auto issue = [&](int slot, int kb) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      if (!A16 && i < LPA) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pipe::dma4(src4[A16 ? 0 : i][j] + (int64_t)kb * 32, dst[i] + slot * kStageBytes + 256 * j);
      } else if (NTAIL && tpart[i]) {
        // (a wave issues 3 more DMAs per stage here than the vmcnt waits
        // count: they then wait for more than they need, never for less)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pipe::dma4(tsrc[NTAIL ? i : 0][j] + (int64_t)kb * tstep, dst[i] + slot * kStageBytes + 256 * j);
      } else {
        pipe::dma16(src[i] + (int64_t)kb * step[i], dst[i] + slot * kStageBytes);
      }
    }
  };


  // fragment addressing (f32x4 units inside a stage)
  const int q0 = kg * NQ;
  int a_off[BLK_M], a_swz[BLK_M];
#pragma unroll
  for (int i = 0; i < BLK_M; ++i) {
    const int trow = (wm * BLK_M + i) * MB + fl;
    a_off[i] = (trow >> 3) * 64 + (trow & 7) * 8;
    a_swz[i] = pipe::a_swizzle(trow);
  }

  // NACC = 2: even and odd k-steps accumulate into separate chains, so a wave
  // always has an independent MFMA to issue; the chains are added at the end
  AccT acc[NACC][BLK_M][BLK_N];
#pragma unroll
  for (int c = 0; c < NACC; ++c)
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
      for (int j = 0; j < BLK_N; ++j)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[c][i][j][r] = 0.0f;

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < KB) issue(s, s);
  {
    // Mid-stage barrier.  Halfway through stage kb every wave waits for its
    // DMAs of stage kb+1 and meets the others; stage kb+S-1 then refills the
    // slot of stage kb-1, which no wave reads any more.  So stage kb+1 is
    // published half a stage before it is needed, and the fragments of its
    // first quads are read during the last MFMAs of stage kb: the MFMA pipes
    // see no barrier or LDS-latency gap at the stage boundary.
    constexpr int QPS = NQ;  // 8-k quads per wave per stage (4, or 2 with two k groups)
    constexpr int HALF = QPS / 2;
    // fragment reads run LA quads ahead of the MFMAs, in NFB buffers: two
    // with four quads a stage (reads of stage kb+1 start after the
    // mid-stage barrier that publishes it), one with two
    constexpr int LA = QPS == 4 ? 2 : 1;
    constexpr int NFB = LA == 2 ? 4 : 2;
    f32x4 af[NFB][BLK_M], bf[NFB][BLK_N];
    auto frag_at = [&](const f32x4* stage, int t, int buf) {
      if constexpr (MI16) {
        // 16-k step t: A chunk 4t + l/16 of row fl; packed B quad l/16,
        // lanes 32t + 16*(block's half of its panel) + fl
        const int sub = lane >> 4;
#pragma unroll
        for (int i = 0; i < BLK_M; ++i) af[buf][i] = stage[a_off[i] + ((4 * t + sub) ^ a_swz[i])];
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) {
          const int bj = wn * BLK_N + j;
          bf[buf][j] = stage[(NA + (bj >> 1) * 4 + sub) * 64 + 32 * t + 16 * (bj & 1) + fl];
        }
        return;
      }
      const int q = q0 + t;
#pragma unroll
      for (int i = 0; i < BLK_M; ++i) af[buf][i] = stage[a_off[i] + ((4 * half + q) ^ a_swz[i])];
#pragma unroll
      for (int j = 0; j < BLK_N; ++j) {
        if constexpr (BRM) {
          // k = 16*half + 4q + e sits in slot 8q + 2e + half: the lane
          // halves read adjacent 128-byte rows
          const float* sf = reinterpret_cast<const float*>(stage) +
                            (NA + (wn * BLK_N + j) * 4) * 256 + (8 * q + half) * 32 + l32;
#pragma unroll
          for (int e = 0; e < 4; ++e) bf[buf][j][e] = sf[64 * e];
        } else {
          bf[buf][j] = stage[(NA + (wn * BLK_N + j) * 4 + q) * 64 + lane];
        }
      }
    };
    if (KB > 0) {
      const int inflight = min(KB - 1, S - 2);  // stages 1 .. S-2 may stay in flight
      if (inflight >= 2)
        pipe::wait_vmcnt<2 * DMAS>();
      else if (inflight == 1)
        pipe::wait_vmcnt<DMAS>();
      else
        pipe::wait_vmcnt<0>();
      pipe::barrier_only();
      frag_at(&lds[0][0], 0, 0);
      if constexpr (LA == 2) frag_at(&lds[0][0], 1, 1);
    }
    for (int kb0 = 0; kb0 < KB; kb0 += S) {
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const int kb = kb0 + u;
        if (kb < KB) {
          const f32x4* cur = &lds[u][0];
          const f32x4* nxt = &lds[(u + 1) % S][0];
#pragma unroll
          for (int t = 0; t < QPS; ++t) {
            const int b = LA == 2 ? t : (t & 1);
            // fragments LA quads ahead; after the last stage this reads a
            // stale slot whose values are never used (no branch around the
            // reads)
            if constexpr (LA == 2) {
              if (t + 2 < QPS)
                frag_at(cur, t + 2, (t + 2) & 3);
              else
                frag_at(nxt, t + 2 - QPS, (t + 2) & 3);
            } else {
              if (t + 1 < QPS)
                frag_at(cur, t + 1, b ^ 1);
              else
                frag_at(nxt, 0, b ^ 1);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
              for (int i = 0; i < BLK_M; ++i)
#pragma unroll
                for (int j = 0; j < BLK_N; ++j) {
                  if constexpr (MI16)
                    acc[e % NACC][i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        af[b][i][e], bf[b][j][e], acc[e % NACC][i][j], 0, 0, 0);
                  else
                    acc[e % NACC][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        af[b][i][e], bf[b][j][e], acc[e % NACC][i][j], 0, 0, 0);
                }
            // interleave the next quad's LDS reads with this quad's MFMAs
            constexpr int NDS = BLK_M + (BRM ? 4 : 1) * BLK_N, NMF = 4 * BLK_M * BLK_N;
            constexpr int NIL = NDS < NMF ? NDS : NMF;
#pragma unroll
            for (int r = 0; r < NIL; ++r) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            if constexpr (NMF > NIL) __builtin_amdgcn_sched_group_barrier(0x008, NMF - NIL, 0);
            if constexpr (NDS > NIL) __builtin_amdgcn_sched_group_barrier(0x100, NDS - NIL, 0);
            if (t == HALF - 1 && kb + 1 < KB) {
              // stages kb+2 .. kb+S-2 may stay in flight (S <= 4: at most one)
              if (S >= 4 && kb + 2 < KB)
                pipe::wait_vmcnt<DMAS>();
              else
                pipe::wait_vmcnt<0>();
              pipe::barrier_only();
              if (kb + S - 1 < KB) issue((u + S - 1) % S, kb + S - 1);
            }
          }
        }
      }
    }
  }

  // K tail (K % 32 != 0): packed rows k >= 32*KT of the full panels are
  // row-major [K - 32*KT, nf] (nf = 32*panels); the partial panel's are rows
  // of its row-major [K, N - nf] region
  if (!MI16 && (K & 31)) {
    const int kf = KT * 32;
    const int64_t nf = (int64_t)32 * panels;
    const int64_t tail_base = nf * kf;
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      const int q = q0 + qi;
      f32x4 af[BLK_M], bf[BLK_N];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = 16 * half + 4 * q + e;
        const bool kin = kf + kk < K;
#pragma unroll
        for (int i = 0; i < BLK_M; ++i) {
          const int row = m0 + (wm * BLK_M + i) * 32 + l32;
          af[i][e] = (kin && row < M) ? A[(int64_t)row * p.lda + kf + kk] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < BLK_N; ++j) {
          const int col = n0 + (wn * BLK_N + j) * 32 + l32;
          if constexpr (BRM)
            bf[j][e] = (kin && col < N) ? B[(int64_t)(kf + kk) * p.ldb + col] : 0.0f;
          else if (NTAIL && col >= nf)
            bf[j][e] = (kin && col < N) ? B[nf * K + (int64_t)(kf + kk) * nt + (col - nf)] : 0.0f;
          else
            bf[j][e] = (kin && col < N) ? B[tail_base + (int64_t)kk * nf + col] : 0.0f;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < BLK_M; ++i)
#pragma unroll
          for (int j = 0; j < BLK_N; ++j) {
            if constexpr (!MI16)
              acc[e % NACC][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                  af[i][e], bf[j][e], acc[e % NACC][i][j], 0, 0, 0);
          }
    }
  }
  if constexpr (NACC == 2) {
#pragma unroll
    for (int i = 0; i < BLK_M; ++i)
#pragma unroll
      for (int j = 0; j < BLK_N; ++j) acc[0][i][j] += acc[1][i][j];
  }

  // fused epilogue over accumulator registers [R0, R1)
  const float* __restrict__ E = p.e ? p.e + z * p.stride_e : nullptr;
  float* __restrict__ C = p.c + z * p.stride_c;
  auto epilogue = [&](auto r0_c, auto r1_c) {
    constexpr int R0 = decltype(r0_c)::value, R1 = decltype(r1_c)::value;
#pragma unroll
    for (int i = 0; i < BLK_M; ++i) {
#pragma unroll
      for (int j = 0; j < BLK_N; ++j) {
        const int col = n0 + (wn * BLK_N + j) * MB + fl;
        if (col >= N) continue;
#pragma unroll
        for (int r = R0; r < R1; ++r) {
          // 32x32 block: register r holds row 8*(r/4) + 4*(l/32) + r%4;
          // 16x16 block: row 4*(l/16) + r
          const int row = m0 + (wm * BLK_M + i) * MB +
                          (MI16 ? 4 * (lane >> 4) + r : 8 * (r >> 2) + 4 * half + (r & 3));
          if (row >= M) continue;
          float v = acc[0][i][j][r];
          if (E) v += E[(int64_t)row * p.lde + col];
          if (p.bias) v += bias_v[j];
          // non-temporal: C goes to memory without filling this XCD's L2,
          // so the end-of-kernel release has no dirty C lines to write back
          __builtin_nontemporal_store(apply_epilogue(v, p.epilogue),
                                      &C[(int64_t)row * p.ldc + col]);
        }
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I8 = std::integral_constant<int, 8>;
  using I16 = std::integral_constant<int, 16>;
  if constexpr (KS == 1) {
    epilogue(I0{}, std::integral_constant<int, NR>{});
  } else {
    // The two k groups hold partial sums of the same outputs.  Group g keeps
    // registers [8g, 8g+8) and hands the other eight to its partner through
    // LDS; each output is then partial(0) + partial(1) whichever wave adds.
    f32x4* xch = &lds[0][0];
    auto slot = [&](int owner, int blk, int u) {
      return ((wt * 2 + owner) * BLK_M * BLK_N + blk) * 2 * 64 + u * 64 + lane;
    };
    auto send = [&](auto g_c) {
      constexpr int G = 1 - decltype(g_c)::value;  // receiver; its registers [8G, 8G+8)
#pragma unroll
      for (int i = 0; i < BLK_M; ++i)
#pragma unroll
        for (int j = 0; j < BLK_N; ++j)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            f32x4 v;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = acc[0][i][j][8 * G + 4 * u + c];
            xch[slot(G, i * BLK_N + j, u)] = v;
          }
    };
    auto receive = [&](auto g_c) {
      constexpr int G = decltype(g_c)::value;
#pragma unroll
      for (int i = 0; i < BLK_M; ++i)
#pragma unroll
        for (int j = 0; j < BLK_N; ++j)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const f32x4 v = xch[slot(G, i * BLK_N + j, u)];
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[0][i][j][8 * G + 4 * u + c] += v[c];
          }
    };
    pipe::block_barrier();  // every wave is done with the pipeline stages
    if (kg == 0)
      send(I0{});
    else
      send(std::integral_constant<int, 1>{});
    pipe::block_barrier();
    if (kg == 0) {
      receive(I0{});
      epilogue(I0{}, I8{});
    } else {
      receive(std::integral_constant<int, 1>{});
      epilogue(I8{}, I16{});
    }
  }
}

// dst[z, i, j] = src[z*s0 + i*s1 + j*s2] over [nz, m, n] (a broadcast bias
// materialised as a GEMM addend; strides of broadcast dims are 0).
__global__ void broadcast3_kernel(const float* __restrict__ src, int64_t s0, int64_t s1,
                                  int64_t s2, int64_t nz, int64_t m, int64_t n,
                                  float* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nz * m * n) return;
  const int64_t j = t % n, i = (t / n) % m, z = t / (m * n);
  dst[t] = src[z * s0 + i * s1 + j * s2];
}

// Packs row-major B[z] (leading dimension ldb, batch stride stride_b, N a
// multiple of 32, rows not 16-byte aligned) into the layout_matmul format at
// dst + z*K*N.  Workgroup (t, g) of 256 threads handles k-block t and the
// n-panels ppw*g .. ppw*g + ppw - 1 (ppw = 1, 2 or 4; fewer at the right
// edge).  It reads the 32 x 32*ppw source block as coalesced row segments,
// transposes it through LDS, and writes each panel's 1 KiB fragment block
// with one 16-byte store per thread: thread (q, lane) of the block holds
// k = 32t + 16*(lane/32) + 4q + e, e = 0..3, at n = 32p + lane%32.  The extra
// workgroup column t = K/32 copies the K-tail rows of its panels into the
// row-major tail region.
__global__ __launch_bounds__(256) void pack_rhs_rowmajor_kernel(const float* __restrict__ src,
                                                                int64_t ldb, int64_t stride_b,
                                                                float* __restrict__ dst,
                                                                int64_t dst_stride, int K,
                                                                int N, int ppw) {
  __shared__ float tile[32][128 + 4];
  const int kb = K >> 5, t = blockIdx.x;
  const int p0 = ppw * (int)blockIdx.y;
  const int np = min(ppw, (N >> 5) - p0);
  const int n0 = 32 * p0, width = 32 * np;
  const float* __restrict__ bz = src + (int64_t)blockIdx.z * stride_b;
  float* __restrict__ dz = dst + (int64_t)blockIdx.z * dst_stride;
  const int tid = threadIdx.x;
  if (t < kb) {
    const int c = tid & 31, r = tid >> 5;
    if (4 * c < width) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = r + 8 * i;
        const float* __restrict__ b = bz + (int64_t)(32 * t + row) * ldb + n0 + 4 * c;
        f32x4 v;
        v[0] = b[0];
        v[1] = b[1];
        v[2] = b[2];
        v[3] = b[3];
        *reinterpret_cast<f32x4*>(&tile[row][4 * c]) = v;
      }
    }
    __syncthreads();
    const int q = tid >> 6, lane = tid & 63;
    const int kk = 16 * (lane >> 5) + 4 * q;
    for (int j = 0; j < np; ++j) {
      const int n = 32 * j + (lane & 31);
      f32x4 v;
      v[0] = tile[kk][n];
      v[1] = tile[kk + 1][n];
      v[2] = tile[kk + 2][n];
      v[3] = tile[kk + 3][n];
      *reinterpret_cast<f32x4*>(dz + ((int64_t)(p0 + j) * kb + t) * 1024 + tid * 4) = v;
    }
    return;
  }
  const int kf = kb * 32;  // K tail rows: row-major [K - kf, N]
  for (int i = tid; i < (K - kf) * width; i += 256) {
    const int k = kf + i / width, n = n0 + i % width;
    dz[(int64_t)N * kf + (int64_t)(k - kf) * N + n] = bz[(int64_t)k * ldb + n];
  }
}

// The N % 32 tail columns [nf, nf + nt) of row-major B into the packed
// format's N-tail region: row-major [K, nt] at offset nf*K of each batch's
// dst_stride floats.
__global__ __launch_bounds__(256) void pack_rhs_tail_kernel(const float* __restrict__ src,
                                                            int64_t ldb, int64_t stride_b,
                                                            float* __restrict__ dst,
                                                            int64_t dst_stride, int64_t K,
                                                            int64_t nf, int nt) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= K * nt) return;
  const int64_t k = i / nt, c = i % nt;
  dst[(int64_t)blockIdx.y * dst_stride + nf * K + i] =
      src[(int64_t)blockIdx.y * stride_b + k * ldb + nf + c];
}

__global__ void pack_rhs_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t K,
                                int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= K * N) return;
  const int64_t k = i / N, n = i % N;
  dst[layout_pack_offset(k, n, K, N)] = src[i];
}

template <int WM, int WN, int BMB, int BNB, bool PACKED>
int launch_tile(const GemmParams& p0, int64_t batch, hipStream_t stream) {
  constexpr int BM = WM * BMB * 32, BN = WN * BNB * 32;
  GemmParams p = p0;
  p.tiles_m = (p.m + BM - 1) / BM;
  p.tiles_n = (p.n + BN - 1) / BN;
  dim3 grid(p.tiles_m * p.tiles_n, 1, (unsigned)batch);
  hipLaunchKernelGGL((gemm_mfma_kernel<WM, WN, BMB, BNB, PACKED>), grid, dim3(kThreads), 0,
                     stream, p);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

template <int WM, int WN, int BMB, int BNB, int S, int NACC, int KS, bool BRM, bool MI16 = false,
          bool NTAIL = false>
int launch_pipe(const GemmParams& p0, int64_t batch, hipStream_t stream) {
  constexpr int BM = WM * BMB * (MI16 ? 16 : 32), BN = WN * BNB * (MI16 ? 16 : 32);
  GemmParams p = p0;
  p.tiles_m = (p.m + BM - 1) / BM;
  p.tiles_n = (p.n + BN - 1) / BN;
  // the kernel numbers (batch, tile) pairs in 32-bit arithmetic
  ANNC_REQUIRE((int64_t)p.tiles_m * p.tiles_n * batch < (int64_t(1) << 31), "GEMM grid too large");
  dim3 grid(p.tiles_m * p.tiles_n, 1, (unsigned)batch);
  const dim3 block(64 * WM * WN * KS);
  if (p.a_vec) {
    if (batch > 1)
      hipLaunchKernelGGL((gemm_packed_pipe_kernel<WM, WN, BMB, BNB, S, NACC, KS, true, BRM, true, MI16, NTAIL>),
                         grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((gemm_packed_pipe_kernel<WM, WN, BMB, BNB, S, NACC, KS, true, BRM, false, MI16, NTAIL>),
                         grid, block, 0, stream, p);
  } else {
    if (batch > 1)
      hipLaunchKernelGGL((gemm_packed_pipe_kernel<WM, WN, BMB, BNB, S, NACC, KS, false, BRM, true, MI16, NTAIL>),
                         grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL(
          (gemm_packed_pipe_kernel<WM, WN, BMB, BNB, S, NACC, KS, false, BRM, false, MI16, NTAIL>), grid,
          block, 0, stream, p);
  }
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

// Packed B with N % 32 == 0 (or, with NTAIL, a partial last panel): the
// LDS-DMA pipeline (16-byte DMAs for A rows that are 16-byte aligned, 4-byte
// DMAs otherwise), 32 k per stage.
// Tile choice: the one whose busiest CU (256 on MI355X) computes the least
// tile area, ceil(tiles / 256) * BM * BN, so that a 1.25-round grid does not
// pay for two full rounds of large tiles.  On a tie between 128x128 and
// 128x64, K > 512 takes 128x128 (fewer operand bytes per MFMA); shorter K
// takes 128x64, whose 3-stage form (72 KiB of LDS) lets two workgroups share
// a CU when there are at least two tiles per CU, hiding each one's ramp and
// store phase under the other's MFMAs (measured: 8% faster at K = 256, 3% at
// K = 512, 3% slower at K = 845).
// ANNC_GEMM_PIPE selects 16x16-block tilings of the packed pipeline for
// one-batch packed GEMMs with K % 32 == 0 (a tuning study; the default
// tiling measured as fast or faster on every configs shape):
//   "mi16"    128x64 tiles of 4 waves (64x32 per wave, one wave a SIMD),
//             64x64 where 128x64 gives fewer than 256 tiles;
//   "mi16w8"  128x64 tiles of 8 waves (32x32 per wave, two a SIMD),
//             64x64 of 8 waves (16x32) likewise.
// Read on every launch, so a process can compare the forms.
int gemm_pipe_choice() {
  const char* v = std::getenv("ANNC_GEMM_PIPE");
  if (!v || !*v) return 0;
  if (std::strcmp(v, "mi16") == 0) return 1;
  if (std::strcmp(v, "mi16w8") == 0) return 2;
  return 0;
}

template <bool BRM, bool NT>
int launch_pipe_tiles(const GemmParams& p, int64_t batch, hipStream_t stream) {
  if constexpr (!BRM && !NT) {
    const int choice = batch == 1 && (p.k & 31) == 0 ? gemm_pipe_choice() : 0;
    if (choice) {
      const bool big = ((int64_t)(p.m + 127) / 128) * ((p.n + 63) / 64) >= 256;
      if (choice == 1)
        return big ? launch_pipe<2, 2, 4, 2, 4, 1, 1, BRM, true>(p, batch, stream)
                   : launch_pipe<2, 2, 2, 2, 4, 1, 1, BRM, true>(p, batch, stream);
      return big ? launch_pipe<4, 2, 2, 2, 4, 1, 1, BRM, true>(p, batch, stream)
                 : launch_pipe<4, 2, 1, 2, 4, 1, 1, BRM, true>(p, batch, stream);
    }
  }
  const int64_t cus = 256;
  auto tiles = [&](int bm, int bn) {
    return ((int64_t)(p.m + bm - 1) / bm) * ((p.n + bn - 1) / bn) * batch;
  };
  // 64x32 tiles, each k-block split over two wave pairs (one wave a SIMD,
  // 48 KiB of LDS, so three workgroups share a CU): where they fill the chip
  // in one round while 64x64 tiles would leave half of it idle (768-1024 rows
  // of a 1024->512 layer: 12.4 us against 19.6), and where up to three of
  // them per CU all run at once while 64x64 tiles would need a second round
  // (3072 rows of 1024->512: 31.0 us against 36.0 in 128x64 tiles)
  // (N < 32, one partial panel: wider tiles would only compute padding)
  if (tiles(64, 32) <= cus || (tiles(64, 64) > cus && tiles(64, 32) <= 3 * cus) ||
      (NT && p.n < 32))
    return launch_pipe<2, 1, 1, 1, 4, 1, 2, BRM, false, NT>(p, batch, stream);
  auto cost = [&](int bm, int bn) { return ceil_div(tiles(bm, bn), cus) * bm * bn; };
  const int64_t c128 = cost(128, 128), c128x64 = cost(128, 64), c64 = cost(64, 64);
  // 256x128 tiles (8 waves of 64x64, 3 stages of 48 KiB: one workgroup a
  // CU) for K > 512 where they cost no more CU rounds of area than the
  // smaller tiles, i.e. from 8192 rows of a 1024-column layer: half the
  // operand bytes per MFMA of 128x128, 1.5-2% faster at 8192-16384 rows
  const int64_t c256 = cost(256, 128);
  if (p.k > 512 && c256 <= c128 && c256 <= c128x64 && c256 <= c64)
    return launch_pipe<4, 2, 2, 2, 3, 1, 1, BRM, false, NT>(p, batch, stream);
  // 64x64 tiles leave one wave per SIMD; split each k-block over two wave
  // groups so every SIMD runs two
  if (c64 < c128x64 && c64 < c128) return launch_pipe<2, 2, 1, 1, 4, 1, 2, BRM, false, NT>(p, batch, stream);
  if (c128 < c128x64 || (c128 == c128x64 && p.k > 512))
    return p.a_vec ? launch_pipe<4, 2, 1, 2, 4, 1, 1, BRM, false, NT>(p, batch, stream)
                   : launch_pipe<4, 2, 1, 2, 3, 1, 1, BRM, false, NT>(p, batch, stream);
  if (tiles(128, 64) >= 2 * cus) return launch_pipe<4, 2, 1, 1, 3, 2, 1, BRM, false, NT>(p, batch, stream);
  return launch_pipe<4, 2, 1, 1, 4, 2, 1, BRM, false, NT>(p, batch, stream);
}

// 4 < N < 32 (one partial panel) with more than one round of 32x32 blocks:
// 64x32 pipelined tiles, whose B blocks load by 4-byte DMAs (any ldb) while
// A streams through the LDS-DMA stages, instead of a second round of the
// small kernel, whose waves each walk a quarter of K over 32 rows.  Same
// box, the two libraries alternating, us: 9216x16x1024 20.8 -> 17.2,
// 16384x16x1024 22.2 -> 18.2, 32768x16x1024 44.7 -> 26.6, 65536x8x256
// 27.8 -> 21.0, 9216x20x845 19.1 -> 14.5, 9216x24x512 12.1 -> 9.9; with one
// round (8192 rows) the small kernel stays ahead (9.6 against 16.6).
bool skinny_pipe(const GemmParams& p, int64_t batch) {
  return p.n > 4 && p.n < 32 && ((int64_t)(p.m + 31) / 32) * batch > 256;
}

// b_rowmajor: B is row-major, read in place, with 16-byte aligned rows
// (p.b_vec) unless N < 32 (then every B block is the partial panel's, loaded
// by 4-byte DMAs); otherwise B is in the layout_matmul packed format.
int launch_packed_pipe(const GemmParams& p, int64_t batch, hipStream_t stream,
                       bool b_rowmajor = false) {
  const bool nt = (p.n & 31) != 0;
  if (nt)
    return b_rowmajor ? launch_pipe_tiles<true, true>(p, batch, stream)
                      : launch_pipe_tiles<false, true>(p, batch, stream);
  return b_rowmajor ? launch_pipe_tiles<true, false>(p, batch, stream)
                    : launch_pipe_tiles<false, false>(p, batch, stream);
}

template <int W, bool PACKED = false>
int launch_small(const GemmParams& p0, int64_t batch, hipStream_t stream) {
  GemmParams p = p0;
  p.tiles_m = (p.m + 31) / 32;
  p.tiles_n = (p.n + 31) / 32;
  // Few 32x32 blocks and a long K (at least 16 k-blocks a wave, or 8 with at
  // most 32 blocks): K split over up to 8 workgroups a block, each split
  // keeping at least 2 k-blocks a wave, so that up to 256 workgroups run;
  // their partial sums meet in a second launch, added in split order.
  // 1x1024x4096: 23.3 -> 8.6 us; 128x1024x4096: 26.7 -> 18.7; 1x512x1024:
  // 7.5 -> 5.9.  With shorter chains the second launch costs more than the
  // split saves (256x512x1024, 128 blocks: 9.4 against 9.0 us; 1x256x512,
  // 4 k-blocks a wave: 5.5 against 4.9).
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * batch;
  const int kf = p.k >> 5;
  int splits = 1;
  if (kf / W >= 16 || (blocks <= 32 && kf / W >= 8))
    while (splits < 8 && blocks * splits * 2 <= 256 && kf / (splits * 2) >= 2 * W) splits *= 2;
  p.part = nullptr;
  if (splits > 1) {
    const size_t bytes = (size_t)splits * batch * p.m * p.n * sizeof(float);
    p.part = static_cast<float*>(stream_workspace(stream, bytes));
    if (!p.part) splits = 1;
  }
  dim3 grid(p.tiles_m * p.tiles_n, splits, (unsigned)batch);
  if (splits > 1) {
    if (p.a_vec)
      hipLaunchKernelGGL((gemm_small_kernel<W, true, PACKED, true>), grid, dim3(64 * W), 0, stream, p);
    else
      hipLaunchKernelGGL((gemm_small_kernel<W, false, PACKED, true>), grid, dim3(64 * W), 0, stream, p);
  } else if (p.a_vec) {
    hipLaunchKernelGGL((gemm_small_kernel<W, true, PACKED>), grid, dim3(64 * W), 0, stream, p);
  } else {
    hipLaunchKernelGGL((gemm_small_kernel<W, false, PACKED>), grid, dim3(64 * W), 0, stream, p);
  }
  ANNC_HIP_TRY(hipGetLastError());
  if (splits > 1) {
    const int64_t total = batch * p.m * p.n;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                       stream, p, splits, batch);
    ANNC_HIP_TRY(hipGetLastError());
  }
  return ANNC_OK;
}

template <bool PACKED>
int launch_gemm(const GemmParams& p, int64_t batch, hipStream_t stream) {
  // Largest tile that still gives every CU a workgroup (256 CUs on MI355X).
  const int64_t cus = 256;
  auto tiles = [&](int bm, int bn) {
    return ((int64_t)(p.m + bm - 1) / bm) * ((p.n + bn - 1) / bn) * batch;
  };
  // Too few 64x64 tiles to occupy the chip, one round of 32x32 blocks, or
  // N < 32 (one 32-column block; the tile kernel would waste most of its
  // 64-column tiles: 16384x16x1024 85 -> 22 us, and 18 us in the pipelined
  // kernel, which annc_hip_gemm picks first beyond one round: skinny_pipe):
  // 32x32 blocks with K split over four waves (eight measured slower at
  // every K)
  if (!PACKED && (tiles(64, 64) < cus / 2 || tiles(32, 32) <= cus || p.n < 32))
    return launch_small<4>(p, batch, stream);
  if (tiles(128, 128) >= cus) return launch_tile<2, 2, 2, 2, PACKED>(p, batch, stream);
  if (tiles(64, 128) >= cus) return launch_tile<2, 2, 1, 2, PACKED>(p, batch, stream);
  return launch_tile<2, 2, 1, 1, PACKED>(p, batch, stream);
}

// N <= 4: 16 lanes per row (row-major or dense B)
int launch_gemv(const GemmParams& p, int64_t batch, hipStream_t s) {
  dim3 grid((unsigned)ceil_div(p.m, kThreads / 16), 1, (unsigned)batch);
  switch (p.n) {
    case 1: hipLaunchKernelGGL(gemv_rows_kernel<1>, grid, dim3(kThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL(gemv_rows_kernel<2>, grid, dim3(kThreads), 0, s, p); break;
    case 3: hipLaunchKernelGGL(gemv_rows_kernel<3>, grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL(gemv_rows_kernel<4>, grid, dim3(kThreads), 0, s, p); break;
  }
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

// Columns [nf, N) of a GEMM whose first nf = N & ~31 columns ran through the
// pipelined kernel: B's tail columns as a row-major [K, N - nf] block at
// b_tail (row stride ldb_tail; batches stride_b apart), and C, the addend
// and the bias from column nf on.  N - nf <= 4 runs the GEMV kernel, wider
// tails the small kernel (one 32-column block).
int launch_n_tail(const GemmParams& p, int64_t nf, const float* b_tail, int64_t ldb_tail,
                  int64_t batch, hipStream_t s) {
  auto aligned16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  GemmParams t = p;
  t.n = p.n - static_cast<int>(nf);
  t.b = b_tail;
  t.ldb = ldb_tail;
  t.c = p.c + nf;
  if (p.e) t.e = p.e + nf;
  if (p.bias) t.bias = p.bias + nf;
  t.b_vec = ldb_tail % 4 == 0 && p.stride_b % 4 == 0 && aligned16(b_tail);
  t.b_dense = ldb_tail == t.n && p.stride_b % 4 == 0 && aligned16(b_tail);
  if (t.n <= 4) return launch_gemv(t, batch, s);
  if (skinny_pipe(t, batch)) return launch_packed_pipe(t, batch, s, /*b_rowmajor=*/true);
  return launch_small<4>(t, batch, s);
}

// ---------------------------------------------------------------------------
// Tower tail: a dense layer on packed weights (K -> N, bias, activation)
// and the N -> 1 scoring layer after it, in one kernel.
//   * A workgroup owns 16 rows and all N columns, so a row's scoring dot
//     needs no other workgroup: no atomics, no second launch, and every
//     row's sums run in one fixed order.  M = 4096 gives 256 workgroups.
//   * NW = N/16 waves; wave w computes the 16-column block w on
//     v_mfma_f32_16x16x4f32.  A 16-k step feeds k = 4*(l/16) + s to lane l
//     at MFMA step s, so one 16-byte read per operand covers 4 steps.
//   * The 16 rows of A sit in LDS whole, written a round at a time: a round
//     is N k-columns of the 16 rows, one float4 per thread, loaded into
//     registers one round ahead, then one barrier.  Row stride K + 8
//     floats: with K + 4 the fragment reads (16 rows, 4 k-chunks) counted
//     0.5 M cycles of LDS bank conflicts per launch, with K + 8 none.
//   * B streams from L2 straight into registers, two k-blocks ahead, with
//     buffer loads: each lane's float4 of the packed format (layout_pack.h)
//     is the operand of 4 MFMA steps.  Every workgroup reads all of B
//     (K*N*4 bytes), twice the operand bytes of a 64x64-tiled layer, and on
//     the 4096x256x512 layer the loop is bound by that stream: global loads
//     instead of buffer loads took 12.1 us against 10.8 us, and deeper
//     prefetch (3 to 6 blocks) was slower as well.
//   * Workgroups of one XCD start at different rounds (rotating the k
//     order), so that XCD's L2 serves different B blocks at a time.
//   * Epilogue: bias and activation per element (optionally stored as the
//     hidden layer), times the score weight, summed over the wave's 16
//     columns by DPP and then over the waves in wave order through LDS;
//     score bias and activation last.
constexpr int kScoreRows = 16;
constexpr int kScoreMaxK = 2048;

template <int NW, int KMAX>
__global__ __launch_bounds__(64 * NW) void dense_score_kernel(
    const float* __restrict__ A, int64_t lda, int M, int K, const float* __restrict__ B,
    const float* __restrict__ bias, int epilogue, const float* __restrict__ w_score,
    const float* __restrict__ bias_score, int score_epilogue, float* __restrict__ H,
    int64_t ldh, float* __restrict__ out, int64_t ldo) {
  constexpr int N = 16 * NW;
  constexpr int T = 64 * NW;   // threads
  constexpr int RK = N;        // k-columns per round: T float4s over 16 rows
  constexpr int BPR = RK / 32; // 32-k blocks per round
  constexpr int TPR = T / 16;  // threads per row in a round
  static_assert(BPR % 2 == 0, "two-block B ring");
  __shared__ __attribute__((aligned(16))) float a_lds[kScoreRows * (KMAX + 8)];
  __shared__ float red[NW][kScoreRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int m0 = blockIdx.x * kScoreRows;
  const int RS = K + 8;
  const int KT = K >> 5;
  const int R = K / RK;
  // visit round r is round (r + ro) % R; ro differs between workgroups of
  // one XCD (workgroups are dealt to the 8 XCDs round-robin)
  const int ro = (int)((blockIdx.x >> 3) % (unsigned)R);

  // this thread's A float4 of every round: row arow_t, k-chunk ac4
  const int arow_t = tid / TPR, ac4 = tid % TPR;
  const float* a_src = A + (int64_t)min(m0 + arow_t, M - 1) * lda + 4 * ac4;
  float* a_dst = a_lds + arow_t * RS + 4 * ac4;

  // B: wave w's 16 columns are half (w & 1) of 32-column panel w/2; lane
  // (g, c) reads the float4 of quad g, lane 16*(w & 1) + c, 16-k half h
  // 128h floats further (layout_pack.h)
  const __amdgpu_buffer_rsrc_t brs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), 0, K * N * 4, 0x00020000);
  const int b_off = ((wave >> 1) * KT * 1024 + 256 * g + 4 * (16 * (wave & 1) + c)) * 4;
  auto load_b = [&](int t, int h) {
    return __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, b_off + (t * 1024 + 128 * h) * 4, 0, 0));
  };

  // epilogue operands of this lane's column 16*wave + c, fetched before the
  // loop rather than after it (11.07 against 11.20 us per launch at
  // 4096x512x256)
  const int col = 16 * wave + c;
  const float bj = bias ? bias[col] : 0.0f;
  const float wj = w_score[col];
  const float b_score = bias_score ? bias_score[0] : 0.0f;

  int ar = ro;  // round being visited
  f32x4 a_next = *reinterpret_cast<const f32x4*>(a_src + ar * RK);
  f32x4 bq[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bq[s][0] = load_b(ar * BPR + s, 0);
    bq[s][1] = load_b(ar * BPR + s, 1);
  }
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const float* a_frag = a_lds + c * RS + 4 * g;
  for (int r = 0; r < R; ++r) {
    const int an = (ar + 1 == R) ? 0 : ar + 1;  // next round visited
    *reinterpret_cast<f32x4*>(a_dst + ar * RK) = a_next;
    if (r + 1 < R) a_next = *reinterpret_cast<const f32x4*>(a_src + an * RK);
    __syncthreads();
#pragma unroll
    for (int tb = 0; tb < BPR; ++tb) {
      const int t = ar * BPR + tb;
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(a_frag + 32 * t);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(a_frag + 32 * t + 16);
      const int s = tb & 1;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[e], bq[s][0][e], acc, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[e], bq[s][1][e], acc, 0, 0, 0);
      // refill this slot with the block visited two blocks later
      if (tb + 2 < BPR) {
        bq[s][0] = load_b(t + 2, 0);
        bq[s][1] = load_b(t + 2, 1);
      } else if (r + 1 < R) {
        const int tn = an * BPR + tb + 2 - BPR;
        bq[s][0] = load_b(tn, 0);
        bq[s][1] = load_b(tn, 1);
      }
    }
    ar = an;
  }

  // rows 4g .. 4g+3, column col of this wave's block
  float part[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = apply_epilogue(acc[r] + bj, epilogue);
    const int row = m0 + 4 * g + r;
    if (H && row < M) __builtin_nontemporal_store(v, H + (int64_t)row * ldh + col);
    float sum = v * wj;
    sum = dpp_add<0x128>(sum);  // row_ror:8
    sum = dpp_add<0x124>(sum);  // row_ror:4
    sum = dpp_add<0x04E>(sum);  // quad_perm [2,3,0,1]
    sum = dpp_add<0x0B1>(sum);  // quad_perm [1,0,3,2]
    part[r] = sum;
  }
  if (c == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * g + r] = part[r];
  }
  __syncthreads();
  if (wave == 0 && lane < kScoreRows) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) sum += red[w][lane];
    if (bias_score) sum += b_score;
    const int row = m0 + lane;
    if (row < M) out[(int64_t)row * ldo] = apply_epilogue(sum, score_epilogue);
  }
}

template <int NW>
void launch_dense_score(hipStream_t s, int kmax, dim3 grid, const float* a, int64_t lda, int m,
                        int k, const float* b, const float* bias, int epilogue,
                        const float* w_score, const float* bias_score, int score_epilogue,
                        float* hidden, int64_t ldh, float* out, int64_t ldo) {
  const dim3 block(64 * NW);
#define ANNC_SCORE_LAUNCH(KMAX)                                                                 \
  hipLaunchKernelGGL((dense_score_kernel<NW, KMAX>), grid, block, 0, s, a, lda, m, k, b, bias, \
                     epilogue, w_score, bias_score, score_epilogue, hidden, ldh, out, ldo)
  if (kmax <= 512)
    ANNC_SCORE_LAUNCH(512);
  else if (kmax <= 1024)
    ANNC_SCORE_LAUNCH(1024);
  else
    ANNC_SCORE_LAUNCH(kScoreMaxK);
#undef ANNC_SCORE_LAUNCH
}

}  // namespace

int launch_broadcast3(hipStream_t s, const float* src, int64_t s0, int64_t s1, int64_t s2,
                      int64_t nz, int64_t m, int64_t n, float* dst) {
  const int64_t total = nz * m * n;
  if (total == 0) return ANNC_OK;
  hipLaunchKernelGGL(broadcast3_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s,
                     src, s0, s1, s2, nz, m, n, dst);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

}  // namespace annc

extern "C" {

int annc_hip_gemm(void* stream, int64_t batch, int64_t m, int64_t n, int64_t k, const float* a,
                  int64_t lda, int64_t stride_a, const float* b, int64_t ldb, int64_t stride_b,
                  int b_packed, const float* addend, int64_t lde, int64_t stride_e,
                  const float* bias, int epilogue, float* c, int64_t ldc, int64_t stride_c) {
  using namespace annc;
  ANNC_REQUIRE(batch >= 0 && m >= 0 && n >= 0 && k >= 0, "negative GEMM dimension");
  ANNC_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31) && batch < 65536,
               "GEMM dimension too large");
  if (batch == 0 || m == 0 || n == 0) return set_error(ANNC_OK, "");
  // packed with N < 32 is row-major [K, N] (no full panels)
  if (b_packed && n < 32) {
    b_packed = 0;
    ldb = n;
  }
  ANNC_REQUIRE(c != nullptr, "null output");
  ANNC_REQUIRE(k == 0 || (a != nullptr && b != nullptr), "null operand");
  ANNC_REQUIRE(b_packed || ldb >= n, "ldb < n");
  ANNC_REQUIRE(lda >= k && ldc >= n, "leading dimension too small");
  ANNC_REQUIRE(addend == nullptr || lde >= n, "lde < n");
  ANNC_REQUIRE((epilogue & ~(ANNC_EPI_RELU | ANNC_EPI_SIGMOID)) == 0, "unknown epilogue bits");
  hipStream_t s = static_cast<hipStream_t>(stream);

  GemmParams p{};
  p.a = a;
  p.b = b;
  p.e = addend;
  p.bias = bias;
  p.c = c;
  p.lda = lda;
  p.ldb = b_packed ? n : ldb;  // packed with N < 32 is row-major [K, N]
  p.lde = lde;
  p.ldc = ldc;
  p.stride_a = stride_a;
  p.stride_b = stride_b;
  p.stride_e = stride_e;
  p.stride_c = stride_c;
  p.m = (int)m;
  p.n = (int)n;
  p.k = (int)k;
  p.epilogue = epilogue;
  auto aligned16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  p.a_vec = (lda % 4 == 0) && (stride_a % 4 == 0) && aligned16(a);
  p.b_vec = (ldb % 4 == 0) && (stride_b % 4 == 0) && aligned16(b);
  p.b_dense = (p.ldb == n) && (stride_b % 4 == 0) && aligned16(b);

  if (n <= 4) {
    const int rc = launch_gemv(p, batch, s);
    return set_error(rc, rc == ANNC_OK ? "" : "GEMV launch failed");
  }
  if (n < 32 && skinny_pipe(p, batch)) return launch_packed_pipe(p, batch, s, /*b_rowmajor=*/true);
  // N % 32 != 0 with more than one round of 32x32 blocks in its full
  // 32-column panels: the pipelined kernel with a partial last panel (B
  // packed, or row-major with 16-byte aligned rows) where the extra column
  // of tiles costs no more CU rounds (one_launch), else the full panels
  // pipelined (row-major B without aligned rows packed per call first) and
  // then the N % 32 tail columns through a small kernel; instead of the tile
  // kernel over all of N.  4096x1000x1024: 122 us -> 78 (two launches) or
  // 73 (one); 4096x520x1024: 123 -> 46 (two; one launch needs a 5th CU
  // round of tiles: 62).
  const int64_t nf = n & ~int64_t(31);
  const bool split_n = n % 32 != 0 && nf > 0 && ceil_div(m, 32) * (nf / 32) * batch > 256;
  // the pipelined kernel's busiest-CU tile area over nn columns, the least
  // over the tilings its launcher picks from
  auto round_area = [&](int64_t nn) {
    static constexpr int kShapes[5][2] = {{256, 128}, {128, 128}, {128, 64}, {64, 64}, {64, 32}};
    int64_t best = INT64_MAX;
    for (const auto& sh : kShapes) {
      if (sh[0] == 256 && k <= 512) continue;
      const int64_t t = ceil_div(m, sh[0]) * ceil_div(nn, sh[1]) * batch;
      best = std::min<int64_t>(best, ceil_div(t, 256) * sh[0] * sh[1]);
    }
    return best;
  };
  const bool one_launch = split_n && round_area(n) <= round_area(nf);
  if (b_packed) {
    ANNC_REQUIRE(aligned16(b) && stride_b % 4 == 0, "packed B must be 16-byte aligned");
    // At most one round of 32x32 blocks (small batches): 32x32 blocks with K
    // split over four waves, as for row-major B, whose results these equal
    // bit for bit (a partial last panel reads the format's N-tail region).
    // At 1-512 rows of configs[1]'s layer 1 this takes 6-8 us against 19 us
    // in the pipelined kernel, whose few workgroups each stream the whole K;
    // 256x1000x1024: 61 -> 10 us against the tile kernel.
    if (ceil_div(m, 32) * ceil_div(n, 32) * batch <= 256) return launch_small<4, true>(p, batch, s);
    if (n % 32 == 0) return launch_packed_pipe(p, batch, s);
    // one launch: the partial last panel from the format's row-major N-tail
    // region; two: the format's first nf*K floats are the packed [K, nf]
    // matrix of the full panels, and the N-tail region follows
    if (round_area(n) <= round_area(nf)) return launch_packed_pipe(p, batch, s);
    GemmParams q = p;
    q.n = static_cast<int>(nf);
    q.ldb = nf;
    const int rc = launch_packed_pipe(q, batch, s);
    if (rc != ANNC_OK) return set_error(rc, "GEMM launch failed");
    return launch_n_tail(p, nf, b + nf * k, n - nf, batch, s);
  }
  // Large row-major-B GEMMs (the __matmul* and __batch_matmul custom calls,
  // whose weights XLA passes row-major) run the LDS-DMA pipeline, about 1.5x
  // faster than the row-major kernel on the tower shapes: in place when B's
  // rows are 16-byte aligned, else after packing B into the stream workspace
  // (8*K*N bytes moved; also below 512 rows: 500x2048x1024 with ldb = 2049
  // takes 28 us against 61 in the tile kernel).
  // Up to one round of 32x32 blocks runs the small kernel (launch_gemm), as
  // for packed B.  N % 32 != 0 (split_n): the first nm = nf columns as below,
  // then the tail columns.
  const int64_t tiles32 = ceil_div(m, 32) * ceil_div(n, 32) * batch;
  const bool whole = n % 32 == 0 && tiles32 > 256;
  if (whole || split_n) {
    if (p.b_vec && (whole || one_launch))
      return launch_packed_pipe(p, batch, s, /*b_rowmajor=*/true);
    const int64_t nm = whole ? n : nf;  // columns through the pipelined kernel
    GemmParams q = p;
    q.n = static_cast<int>(nm);
    auto then_tail = [&](int rc) -> int {
      if (rc != ANNC_OK || nm == n) return rc;
      return launch_n_tail(p, nm, b + nm, ldb, batch, s);
    };
    if (p.b_vec) return then_tail(launch_packed_pipe(q, batch, s, /*b_rowmajor=*/true));
    const int64_t tiles64 = ceil_div(m, 64) * ceil_div(nm, 64) * batch;
    // each batch's packed matrix starts 16-byte aligned (the packed kernels'
    // 16-byte DMAs)
    const int64_t bstride = (k * n + 3) & ~int64_t(3);
    const int64_t packed_bytes = batch * bstride * static_cast<int64_t>(sizeof(float));
    if (tiles64 >= 128 && packed_bytes <= (int64_t(1) << 31)) {
      float* bp = static_cast<float*>(stream_workspace(s, static_cast<size_t>(packed_bytes)));
      if (bp) {
        // B into the layout_matmul format, which then runs as packed B.  Where
        // the partial panel costs no extra CU round of tiles (one_launch) the
        // tail columns go into the format's row-major N-tail region too and
        // run in the same launch, instead of a second launch that streams A
        // again; otherwise the full panels run, then the tail columns from
        // B itself (a copy would only add a launch).
        // Panels per workgroup: the widest that still gives >= 512 workgroups.
        const int64_t kcols = (k >> 5) + ((k & 31) ? 1 : 0), panels = nm >> 5;
        int ppw = 4;
        while (ppw > 1 && kcols * ceil_div(panels, ppw) * batch < 512) ppw >>= 1;
        const dim3 grid((unsigned)kcols, (unsigned)ceil_div(panels, ppw), (unsigned)batch);
        hipLaunchKernelGGL(pack_rhs_rowmajor_kernel, grid, dim3(256), 0, s, b, ldb, stride_b, bp,
                           bstride, (int)k, (int)nm, ppw);
        ANNC_HIP_TRY(hipGetLastError());
        if (nm < n && one_launch) {
          const dim3 tgrid((unsigned)ceil_div(k * (n - nm), 256), (unsigned)batch);
          hipLaunchKernelGGL(pack_rhs_tail_kernel, tgrid, dim3(256), 0, s, b, ldb, stride_b, bp,
                             bstride, k, nm, (int)(n - nm));
          ANNC_HIP_TRY(hipGetLastError());
        }
        GemmParams r = p;
        r.b = bp;
        r.ldb = n;
        r.stride_b = bstride;
        if (nm == n || one_launch) return launch_packed_pipe(r, batch, s);
        GemmParams f = r;
        f.n = static_cast<int>(nm);
        f.ldb = nm;
        return then_tail(launch_packed_pipe(f, batch, s));
      }
    }
  }
  return launch_gemm<false>(p, batch, s);
}

int annc_hip_layout_matmul_pack_rhs(void* stream, int64_t k, int64_t n, const float* src,
                                    float* dst) {
  using namespace annc;
  ANNC_REQUIRE(k >= 0 && n >= 0, "negative dimension");
  ANNC_REQUIRE(src != nullptr && dst != nullptr && src != dst, "bad pointers");
  const int64_t total = k * n;
  if (total == 0) return set_error(ANNC_OK, "");
  hipLaunchKernelGGL(pack_rhs_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, dst, k, n);
  ANNC_HIP_TRY(hipGetLastError());
  return set_error(ANNC_OK, "");
}

int annc_hip_dense_score(void* stream, int64_t m, int64_t n, int64_t k, const float* a,
                         int64_t lda, const float* b_packed, const float* bias, int epilogue,
                         const float* w_score, const float* bias_score, int score_epilogue,
                         float* hidden, int64_t ldh, float* out, int64_t ldo) {
  using namespace annc;
  auto aligned16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  ANNC_REQUIRE(m >= 0 && m < (1ll << 31) - kScoreRows, "bad row count");
  ANNC_REQUIRE(n == 64 || n == 128 || n == 256, "dense_score: n must be 64, 128 or 256");
  ANNC_REQUIRE(k >= n && k <= kScoreMaxK && k % n == 0,
               "dense_score: k must be a multiple of n, at most %d", kScoreMaxK);
  ANNC_REQUIRE((epilogue & ~(ANNC_EPI_RELU | ANNC_EPI_SIGMOID)) == 0 &&
                   (score_epilogue & ~(ANNC_EPI_RELU | ANNC_EPI_SIGMOID)) == 0,
               "unknown epilogue bits");
  if (m == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(a != nullptr && b_packed != nullptr && w_score != nullptr && out != nullptr,
               "null operand");
  ANNC_REQUIRE(lda >= k && lda % 4 == 0 && aligned16(a), "A rows must be 16-byte aligned");
  ANNC_REQUIRE(aligned16(b_packed), "packed B must be 16-byte aligned");
  ANNC_REQUIRE(ldo >= 1, "bad output stride");
  ANNC_REQUIRE(hidden == nullptr || ldh >= n, "ldh < n");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)ceil_div(m, kScoreRows));
  const int mi = (int)m, ki = (int)k, kmax = (int)k;
  switch (n) {
    case 64:
      launch_dense_score<4>(s, kmax, grid, a, lda, mi, ki, b_packed, bias, epilogue, w_score,
                            bias_score, score_epilogue, hidden, ldh, out, ldo);
      break;
    case 128:
      launch_dense_score<8>(s, kmax, grid, a, lda, mi, ki, b_packed, bias, epilogue, w_score,
                            bias_score, score_epilogue, hidden, ldh, out, ldo);
      break;
    default:
      launch_dense_score<16>(s, kmax, grid, a, lda, mi, ki, b_packed, bias, epilogue, w_score,
                             bias_score, score_epilogue, hidden, ldh, out, ldo);
      break;
  }
  ANNC_HIP_TRY(hipGetLastError());
  return set_error(ANNC_OK, "");
}

}  // extern "C"
