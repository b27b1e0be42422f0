// gemv_mt_q4_0.hip -- the several-token matrix-core GEMV kernels for Q4_0 blocks (gemv_mt.hpp).
#include "gemv_mt.hpp"

WH_GEMV_MT_LAUNCHER(q4_0, WH_TYPE_Q4_0)
