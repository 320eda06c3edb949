// gemm_mid_ex.hip -- the mid-size GEMM kernel's fused-epilogue instances (f16 / bf16 inputs; fp32,
// f16 or bf16 D), in a translation unit of their own so that they compile beside the plain ones.
#include "gemm_mid_kernel.hpp"

namespace lava {

LAVA_MID_LAUNCH_INST(f16, float, true)
LAVA_MID_LAUNCH_INST(f16, f16, true)
LAVA_MID_LAUNCH_INST(f16, bf16, true)
LAVA_MID_LAUNCH_INST(bf16, float, true)
LAVA_MID_LAUNCH_INST(bf16, f16, true)
LAVA_MID_LAUNCH_INST(bf16, bf16, true)

}  // namespace lava
