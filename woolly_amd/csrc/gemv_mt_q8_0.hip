// gemv_mt_q8_0.hip -- the several-token matrix-core GEMV kernels for Q8_0 blocks (gemv_mt.hpp).
#include "gemv_mt.hpp"

WH_GEMV_MT_LAUNCHER(q8_0, WH_TYPE_Q8_0)
