// pack.cpp -- host side of the layout_matmul pre-pack (the annc-opt step,
// python/annc/optimize/constant_folding.py:77-88), emitting the MFMA
// fragment order described in layout_pack.h instead of kpgemm "kn4" panels.
#include <cstring>

#include "annc_hip.h"
#include "layout_pack.h"

extern "C" {

const char* annc_layout_matmul_rhs_format(void) { return "mfma_f32_32x32x2_k16"; }

int annc_layout_matmul_pack_rhs(int64_t k, int64_t n, const float* src, float* dst) {
  if (k < 0 || n < 0 || (k * n > 0 && (!src || !dst)) || (src == dst && k * n > 0))
    return ANNC_INVALID_ARGUMENT;
  for (int64_t kk = 0; kk < k; ++kk)
    for (int64_t nn = 0; nn < n; ++nn) dst[annc::layout_pack_offset(kk, nn, k, n)] = src[kk * n + nn];
  return ANNC_OK;
}

int annc_layout_matmul_unpack_rhs(int64_t k, int64_t n, const float* src, float* dst) {
  if (k < 0 || n < 0 || (k * n > 0 && (!src || !dst)) || (src == dst && k * n > 0))
    return ANNC_INVALID_ARGUMENT;
  for (int64_t kk = 0; kk < k; ++kk)
    for (int64_t nn = 0; nn < n; ++nn) dst[kk * n + nn] = src[annc::layout_pack_offset(kk, nn, k, n)];
  return ANNC_OK;
}

}  // extern "C"
