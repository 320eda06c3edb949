// gemm_mid_ex.hip -- the mid-size GEMM kernel's fused-epilogue instances (f16 / bf16 inputs; fp32,
// f16 or bf16 D) and its unsigned-byte instance (uint32 product in int32 words), in a translation
// unit of their own so that they compile beside the plain ones.
#include "gemm_mid_kernel.hpp"

namespace lava {

LAVA_MID_LAUNCH_INST(f16, float, true, false)
LAVA_MID_LAUNCH_INST(f16, f16, true, false)
LAVA_MID_LAUNCH_INST(f16, bf16, true, false)
LAVA_MID_LAUNCH_INST(bf16, float, true, false)
LAVA_MID_LAUNCH_INST(bf16, f16, true, false)
LAVA_MID_LAUNCH_INST(bf16, bf16, true, false)
LAVA_MID_LAUNCH_INST(int8_t, int32_t, false, true)

}  // namespace lava
