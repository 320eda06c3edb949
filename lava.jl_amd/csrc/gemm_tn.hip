// gemm_tn.hip -- the compute-bound GEMM: eligibility, the layout dispatcher and the
// instances with both operands K-contiguous (A row-major, B column-major: the bf16 and
// int8 configurations).  The kernel (gemm_tn16_kernel) is
// gemm_tn_kernel.hpp; the other operand forms are instantiated in gemm_tn_{nk,kn,nn}.hip.
#include "gemm_tn_kernel.hpp"

namespace lava {

LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_EXTERN, false, true)
LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_EXTERN, true, false)
LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_EXTERN, false, false)
LAVA_TN_LAYOUT_EXTERN(int8_t, int32_t, false, false, true)
LAVA_TN_LAYOUT_EXTERN(int8_t, int32_t, false, true, false)
LAVA_TN_LAYOUT_EXTERN(int8_t, int32_t, false, false, false)

LAVA_TN_LAYOUT_U8_EXTERN(false, true)
LAVA_TN_LAYOUT_U8_EXTERN(true, false)
LAVA_TN_LAYOUT_U8_EXTERN(false, false)

LAVA_TN_LAYOUT_16BIT(LAVA_TN_LAYOUT_INST, true, true)
LAVA_TN_LAYOUT_INST(int8_t, int32_t, false, true, true)
LAVA_TN_LAYOUT_U8_INST(true, true)

// The unsigned 8-bit product on the tile kernel (bytes in int8_t storage), any operand form.
int launch_gemm_tn_u8(const int8_t* A, const int8_t* B, int32_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc, hipStream_t s, bool ragged, bool ak, bool bk) {
    const Epilogue none{};
    if (ak && bk)
        return launch_gemm_tn_layout<int8_t, int32_t, false, true, true, true>(A, B, C, M, N, K, lda, ldb, ldc, s, none,
                                                                                ragged);
    if (!ak && bk)
        return launch_gemm_tn_layout<int8_t, int32_t, false, false, true, true>(A, B, C, M, N, K, lda, ldb, ldc, s, none,
                                                                                 ragged);
    if (ak && !bk)
        return launch_gemm_tn_layout<int8_t, int32_t, false, true, false, true>(A, B, C, M, N, K, lda, ldb, ldc, s, none,
                                                                                 ragged);
    return launch_gemm_tn_layout<int8_t, int32_t, false, false, false, true>(A, B, C, M, N, K, lda, ldb, ldc, s, none,
                                                                              ragged);
}

template <typename T, typename OutT, bool EPI>
int launch_gemm_tn(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                   int64_t ldc, hipStream_t s, const Epilogue& epi, bool ragged, bool ak, bool bk) {
    if (ak && bk) return launch_gemm_tn_layout<T, OutT, EPI, true, true>(A, B, C, M, N, K, lda, ldb, ldc, s, epi, ragged);
    if (!ak && bk)
        return launch_gemm_tn_layout<T, OutT, EPI, false, true>(A, B, C, M, N, K, lda, ldb, ldc, s, epi, ragged);
    if (ak && !bk)
        return launch_gemm_tn_layout<T, OutT, EPI, true, false>(A, B, C, M, N, K, lda, ldb, ldc, s, epi, ragged);
    return launch_gemm_tn_layout<T, OutT, EPI, false, false>(A, B, C, M, N, K, lda, ldb, ldc, s, epi, ragged);
}

template int tn_gemm_eligible<f16>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t, int64_t,
                                   int64_t, size_t, bool, bool);
template int tn_gemm_eligible<bf16>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t,
                                    int64_t, int64_t, size_t, bool, bool);
template int tn_gemm_eligible<int8_t>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t,
                                      int64_t, int64_t, size_t, bool, bool);
#define LAVA_TN_INST(T, O, E)                                                                                      \
    template int launch_gemm_tn<T, O, E>(const T*, const T*, O*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, \
                                         hipStream_t, const Epilogue&, bool, bool, bool);
LAVA_TN_INST(f16, float, false)
LAVA_TN_INST(bf16, float, false)
LAVA_TN_INST(int8_t, int32_t, false)
LAVA_TN_INST(f16, float, true)
LAVA_TN_INST(f16, f16, true)
LAVA_TN_INST(f16, bf16, true)
LAVA_TN_INST(bf16, float, true)
LAVA_TN_INST(bf16, f16, true)
LAVA_TN_INST(bf16, bf16, true)
#undef LAVA_TN_INST

}  // namespace lava
