// gemv_mt_q4_k.hip -- the several-token matrix-core GEMV kernels for Q4_K blocks (gemv_mt.hpp).
#include "gemv_mt.hpp"

WH_GEMV_MT_LAUNCHER(q4_k, WH_TYPE_Q4_K)
