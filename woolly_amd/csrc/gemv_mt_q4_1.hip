// gemv_mt_q4_1.hip -- the several-token matrix-core GEMV kernels for Q4_1 blocks (gemv_mt.hpp).
#include "gemv_mt.hpp"

WH_GEMV_MT_LAUNCHER(q4_1, WH_TYPE_Q4_1)
