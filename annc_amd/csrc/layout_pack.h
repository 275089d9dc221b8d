// layout_pack.h -- the layout_matmul pre-packed weight format.
//
// A row-major weight W[K, N] is re-ordered into exactly K*N floats (the
// reference re-saves packed variables in their original shape,
// python/annc/optimize/constant_folding.py:85 and data_pack.py:41):
//
//   region 1  [0, nf*kf)          full 32x32 (k, n) blocks, block (p, t) at
//                                 (p*(kf/32) + t)*1024 for n-panel p and
//                                 k-block t; inside a block the float at
//                                 q*256 + lane*4 + e holds
//                                   k = 32t + 16*(lane/32) + 4q + e,
//                                   n = 32p + lane%32,
//                                 i.e. the B operand of 16 consecutive
//                                 v_mfma_f32_32x32x2f32 steps, one 16-byte
//                                 load per lane per 4 steps, fully coalesced;
//   region 2  [nf*kf, nf*K)       the K tail rows (k >= kf) of the full
//                                 panels, row-major [K-kf, nf];
//   region 3  [nf*K, K*N)         the N tail columns (n >= nf), row-major
//                                 [K, N-nf]  (for N < 32 this is W itself).
//
// kf = K rounded down to 32, nf = N rounded down to 32.  Format tag:
// "mfma_f32_32x32x2_k16".
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define ANNC_HD __host__ __device__
#else
#define ANNC_HD
#endif

namespace annc {

ANNC_HD inline int64_t layout_pack_offset(int64_t k, int64_t n, int64_t K, int64_t N) {
  const int64_t kf = K & ~int64_t(31);
  const int64_t nf = N & ~int64_t(31);
  if (n >= nf) return nf * K + k * (N - nf) + (n - nf);
  if (k >= kf) return nf * kf + (k - kf) * nf + n;
  const int64_t p = n >> 5, j = n & 31;
  const int64_t t = k >> 5, kk = k & 31;
  const int64_t h = kk >> 4, s = kk & 15;
  const int64_t lane = h * 32 + j;
  return (p * (kf >> 5) + t) * 1024 + (s >> 2) * 256 + lane * 4 + (s & 3);
}

}  // namespace annc
