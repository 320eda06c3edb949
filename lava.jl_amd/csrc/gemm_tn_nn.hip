// gemm_tn_nn.hip -- tile-kernel instances for A column-major (M-contiguous), B row-major (N-contiguous).
#include "gemm_tn_kernel.hpp"

namespace lava {

LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_INST, false, false)
LAVA_TN_LAYOUT_INST(int8_t, int32_t, false, false, false)
LAVA_TN_LAYOUT_U8_INST(false, false)

}  // namespace lava
