// gemm_tn_kn.hip -- tile-kernel instances for A row-major (K-contiguous), B row-major (N-contiguous): the coopmat2 and fp16-256 layout.
#include "gemm_tn_kernel.hpp"

namespace lava {

LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_INST, true, false)
LAVA_TN_LAYOUT_INST(int8_t, int32_t, false, true, false)
LAVA_TN_LAYOUT_U8_INST(true, false)

}  // namespace lava
