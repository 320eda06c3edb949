// gemm_tn_nk.hip -- tile-kernel instances for A column-major (M-contiguous), B column-major (K-contiguous).
#include "gemm_tn_kernel.hpp"

namespace lava {

LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_INST, false, true)
LAVA_TN_LAYOUT_INST(int8_t, int32_t, false, false, true)
LAVA_TN_LAYOUT_U8_INST(false, true)

}  // namespace lava
