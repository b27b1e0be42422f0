// gemm.hip -- quantized matrix-matrix product Y = X W^T on gfx950.
#include "wh_blocks.hpp"

namespace wh {

// Y[t, r] = sum_k X[t, k] W[r, k].  Each token row is one GEMV.
int launch_gemm(int type, const void* w, size_t n_rows, size_t k, const float* x, size_t n_tokens,
                float* y, hipStream_t s) {
  for (size_t t = 0; t < n_tokens; t++) {
    int st = launch_gemv(type, w, x + t * k, y + t * n_rows, n_rows, k, s);
    if (st != WH_OK) return st;
  }
  return WH_OK;
}

}  // namespace wh
