// gemv_mt_q6_k.hip -- the several-token matrix-core GEMV kernels for Q6_K blocks (gemv_mt.hpp).
#include "gemv_mt.hpp"

WH_GEMV_MT_LAUNCHER(q6_k, WH_TYPE_Q6_K)
