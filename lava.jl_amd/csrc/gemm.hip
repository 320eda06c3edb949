// gemm.hip -- GEMM entry points: argument checks and kernel choice.
//
// A column-major C is handled as its row-major transpose, C^T = B^T A^T, which
// swaps the operands and flips their layouts; so every kernel writes row-major C.
// Compute-bound shapes take the 256 x 256 tile kernel (gemm_tn_kernel.hpp) in any
// operand layout (K-contiguous operands read directly, M/N-contiguous ones through
// transposing LDS reads, 16- or 8-bit) -- whole tiles, or ragged extents with
// zero-clamped loads.  Mid-size products, plain or with the fused epilogue (at least 128 tiles of
// 128 x 128 and fewer than 144 of 256 x 256, or 257 to 336 of them: mid_gemm_preferred), take the
// 128 x 128 kernel (gemm_mid_kernel.hpp).  Other products of at most 16
// tiles of 256 x 256, and products that the tile kernel would run on few CUs or mostly empty
// tiles (small_gemm_preferred's rate estimate), take the 64 x 64 small-product kernel (with K
// split over the stream's workspace where its tiles alone would leave CUs idle:
// small_gemm_splits); the rest (extents that split a 16-byte chunk) the staged kernel.  Unsigned bytes (lava_hip_gemm_u8_u32) take the same choice among the tile and small
// kernels' unsigned forms, and a one-thread-per-element kernel where the staged kernel would run.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "gemm_kernels.hpp"
#include "lava_hip_internal.hpp"

using namespace lava;

namespace {

// U8: int8 storage read as unsigned bytes, uint32 results (the int32 words' bits); the same
// kernel choice, with each kernel's unsigned form and a one-thread-per-element kernel in the
// staged kernel's place.
template <typename T, typename OutT = typename Mfma16<T>::acc_elem, bool EPI = false, bool U8 = false>
int gemm_entry(const char* name, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
               int64_t ldb, int64_t ldc, uint32_t layout, void* stream, Epilogue epi = Epilogue{}) {
    static_assert(!U8 || (std::is_same<T, int8_t>::value && !EPI), "unsigned: int8 storage, no epilogue");
    using Acc = OutT;
    LAVA_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative extent (M=%lld N=%lld K=%lld)", name, (long long)M,
             (long long)N, (long long)K);
    LAVA_ARG(layout <= 7u, "%s: layout %u has bits beyond A/B/C row-major", name, layout);
    if (M == 0 || N == 0) return LAVA_HIP_OK;
    LAVA_ARG(C != nullptr, "%s: null C", name);
    LAVA_ARG(K == 0 || (A != nullptr && B != nullptr), "%s: null A or B", name);
    bool arow = layout & 1u, brow = layout & 2u;
    const bool crow = layout & 4u;
    const int64_t k1 = K > 0 ? K : 1;
    LAVA_ARG(lda >= (arow ? k1 : M), "%s: lda = %lld is smaller than %s", name, (long long)lda, arow ? "K" : "M");
    LAVA_ARG(ldb >= (brow ? N : k1), "%s: ldb = %lld is smaller than %s", name, (long long)ldb, brow ? "N" : "K");
    LAVA_ARG(ldc >= (crow ? N : M), "%s: ldc = %lld is smaller than %s", name, (long long)ldc, crow ? "N" : "M");
    LAVA_ARG(aligned(A, sizeof(T)) && aligned(B, sizeof(T)) && aligned(C, sizeof(Acc)),
             "%s: operands not aligned to their element size", name);
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;

    const T* a = static_cast<const T*>(A);
    const T* b = static_cast<const T*>(B);
    if (!crow) {   // C^T = B^T A^T, row-major
        const T* t = a;
        a = b;
        b = t;
        const int64_t tm = M;
        M = N;
        N = tm;
        const int64_t tl = lda;
        lda = ldb;
        ldb = tl;
        const bool ar = arow;
        arow = !brow;
        brow = !ar;
        // the kernels now write D^T: the per-m bias runs along its columns; the residual,
        // column-major like D, is read as its row-major transpose with the same ldr
        epi.bias_on_cols = 1;
    }
    hipStream_t s = as_stream(stream);
    Acc* c = static_cast<Acc*>(C);
    // A kernel pinned by lava_hip_set_kernel_override (tests, A/B timing) runs where it fits.
    const int pin = kernel_override(LAVA_HIP_FAMILY_GEMM);
    const bool small_fits = small_gemm_fits<T>(a, b, M, N, K, lda, ldb, arow, brow);
    const int fit = tn_gemm_eligible<T>(a, b, c, M, N, K, lda, ldb, ldc, sizeof(OutT), arow, !brow);
    // the 128 x 128 mid-size kernel: plain output, the fused epilogue (f16 / bf16) or unsigned bytes
    if constexpr (EPI || std::is_same<OutT, typename Mfma16<T>::acc_elem>::value) {
        const int mfit = mid_gemm_eligible<T>(a, b, c, M, N, K, lda, ldb, ldc, sizeof(OutT), arow, !brow);
        if (mfit != TN_NO && (pin == 4 || (pin == 0 && mid_gemm_preferred(M, N))))
            return launch_gemm_mid<T, OutT, EPI, U8>(a, b, c, M, N, K, lda, ldb, ldc, s, epi, mfit == TN_RAGGED, arow,
                                                     !brow);
    }
    bool use_small;
    if (pin == 2)
        use_small = small_fits;
    else if (pin == 3 || (pin == 1 && fit != TN_NO))
        use_small = false;
    else
        use_small = small_fits && small_gemm_preferred<T>(M, N, K);
    if (use_small) {
        if constexpr (!EPI) {
            const SmallSplit sp = pin == 2 ? SmallSplit{} : small_gemm_splits<T>(M, N, K);
            // under graph capture, split only within the workspace the stream already has
            if (sp.splits > 1 && small_splitk_bytes<T>(M, N, sp) <= stream_workspace_cap(stream))
                return launch_gemm_small_splitk<T, U8>(a, b, c, M, N, K, lda, ldb, ldc, arow, brow, stream, sp);
        }
        if constexpr (U8)
            return launch_gemm_small_u8(a, b, c, M, N, K, lda, ldb, ldc, arow, brow, s);
        else
            return launch_gemm_small<T, OutT, EPI>(a, b, c, M, N, K, lda, ldb, ldc, arow, brow, s, epi);
    }
    if (fit != TN_NO && pin != 3) {
        if constexpr (U8)
            return launch_gemm_tn_u8(a, b, c, M, N, K, lda, ldb, ldc, s, fit == TN_RAGGED, arow, !brow);
        else
            return launch_gemm_tn<T, OutT, EPI>(a, b, c, M, N, K, lda, ldb, ldc, s, epi, fit == TN_RAGGED, arow, !brow);
    }
    if constexpr (U8) {
        LAVA_REQUIRE((M * N + 255) / 256 <= 0x7fffffff, LAVA_HIP_ERR_UNSUPPORTED, "%s: problem too large", name);
        return launch_gemm_u8_generic(reinterpret_cast<const uint8_t*>(a), reinterpret_cast<const uint8_t*>(b),
                                      reinterpret_cast<uint32_t*>(c), M, N, K, lda, ldb, ldc,
                                      (arow ? 1u : 0u) | (brow ? 2u : 0u) | 4u, s);
    }
    LAVA_REQUIRE((N + 63) / 64 <= 0x7fffffff && (M + 63) / 64 <= 65535, LAVA_HIP_ERR_UNSUPPORTED,
                 "%s: too many 64-row tiles for the staged kernel (M=%lld N=%lld)", name, (long long)M, (long long)N);
    return launch_gemm_staged<T, OutT, EPI>(a, b, c, M, N, K, lda, ldb, ldc, arow, brow, s, epi);
}

template <typename T, typename OutT>
int gemm_ex_entry(const void* A, const void* B, void* D, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                  int64_t ldd, uint32_t layout, const float* bias, const float* residual, int64_t ldr, int act,
                  void* stream) {
    LAVA_ARG(act >= EPI_NONE && act <= EPI_GELU_ERF, "gemm_ex: unknown activation %d", act);
    LAVA_ARG(aligned(bias, 4) && aligned(residual, 4), "gemm_ex: bias / residual not 4-byte aligned");
    if (residual != nullptr && M > 0 && N > 0)
        LAVA_ARG(ldr >= ((layout & 4u) ? N : M), "gemm_ex: ldr = %lld is smaller than %s", (long long)ldr,
                 (layout & 4u) ? "N" : "M");
    Epilogue epi;
    epi.bias = bias;
    epi.residual = residual;
    epi.ldr = ldr;
    epi.act = act;
    epi.vec4 = aligned(bias, 16) && aligned(residual, 16) && ldr % 4 == 0;
    return gemm_entry<T, OutT, true>("gemm_ex", A, B, D, M, N, K, lda, ldb, ldd, layout, stream, epi);
}

}  // namespace

extern "C" {

int lava_hip_gemm_f16_f32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t layout, void* stream) {
    return gemm_entry<f16>("gemm_f16_f32", A, B, C, M, N, K, lda, ldb, ldc, layout, stream);
}

int lava_hip_gemm_bf16_f32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                           int64_t ldb, int64_t ldc, uint32_t layout, void* stream) {
    return gemm_entry<bf16>("gemm_bf16_f32", A, B, C, M, N, K, lda, ldb, ldc, layout, stream);
}

int lava_hip_gemm_i8_i32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, uint32_t layout, void* stream) {
    return gemm_entry<int8_t>("gemm_i8_i32", A, B, C, M, N, K, lda, ldb, ldc, layout, stream);
}

int lava_hip_gemm_u8_u32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, uint32_t layout, void* stream) {
    return gemm_entry<int8_t, int32_t, false, true>("gemm_u8_u32", A, B, C, M, N, K, lda, ldb, ldc, layout, stream);
}

int lava_hip_gemm_ex(int ab_dtype, int d_dtype, const void* A, const void* B, void* D, int64_t M, int64_t N,
                     int64_t K, int64_t lda, int64_t ldb, int64_t ldd, uint32_t layout, const float* bias,
                     const float* residual, int64_t ldr, int act, void* stream) {
    LAVA_ARG(ab_dtype == LAVA_HIP_F16 || ab_dtype == LAVA_HIP_BF16, "gemm_ex: A/B dtype %d is not f16 or bf16",
             ab_dtype);
    LAVA_ARG(d_dtype == LAVA_HIP_F32 || d_dtype == LAVA_HIP_F16 || d_dtype == LAVA_HIP_BF16,
             "gemm_ex: D dtype %d is not f32, f16 or bf16", d_dtype);
    const bool h = ab_dtype == LAVA_HIP_F16;
    if (d_dtype == LAVA_HIP_F32)
        return h ? gemm_ex_entry<f16, float>(A, B, D, M, N, K, lda, ldb, ldd, layout, bias, residual, ldr, act, stream)
                 : gemm_ex_entry<bf16, float>(A, B, D, M, N, K, lda, ldb, ldd, layout, bias, residual, ldr, act, stream);
    if (d_dtype == LAVA_HIP_F16)
        return h ? gemm_ex_entry<f16, f16>(A, B, D, M, N, K, lda, ldb, ldd, layout, bias, residual, ldr, act, stream)
                 : gemm_ex_entry<bf16, f16>(A, B, D, M, N, K, lda, ldb, ldd, layout, bias, residual, ldr, act, stream);
    return h ? gemm_ex_entry<f16, bf16>(A, B, D, M, N, K, lda, ldb, ldd, layout, bias, residual, ldr, act, stream)
             : gemm_ex_entry<bf16, bf16>(A, B, D, M, N, K, lda, ldb, ldd, layout, bias, residual, ldr, act, stream);
}

int lava_hip_coopmat_gemm_f16_tiles(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                                    int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout, void* stream) {
    LAVA_ARG(M >= 0 && N >= 0 && K >= 0, "coopmat_gemm_f16_tiles: negative extent");
    LAVA_ARG(M % 16 == 0 && N % 16 == 0 && K % 16 == 0,
             "coopmat_gemm_f16_tiles: M, N, K must be multiples of the 16x16x16 tile (M=%lld N=%lld K=%lld)",
             (long long)M, (long long)N, (long long)K);
    LAVA_ARG(layout <= 7u, "coopmat_gemm_f16_tiles: layout %u has bits beyond A/B/C row-major", layout);
    if (M == 0 || N == 0) return LAVA_HIP_OK;
    LAVA_ARG(C != nullptr && (K == 0 || (A != nullptr && B != nullptr)), "coopmat_gemm_f16_tiles: null pointer");
    const bool arow = layout & 1u, brow = layout & 2u, crow = layout & 4u;
    const int64_t k1 = K > 0 ? K : 1;
    LAVA_ARG(lda >= (arow ? k1 : M) && ldb >= (brow ? N : k1) && ldc >= (crow ? N : M),
             "coopmat_gemm_f16_tiles: leading dimension too small");
    LAVA_ARG(aligned(A, 2) && aligned(B, 2) && aligned(C, 4), "coopmat_gemm_f16_tiles: misaligned operand");
    LAVA_ARG((M / 16) * (N / 16) / 4 < 0x7fffffff, "coopmat_gemm_f16_tiles: too many tiles");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    return launch_coopmat_tiles(static_cast<const f16*>(A), static_cast<const f16*>(B), static_cast<float*>(C), M, N,
                                K, lda, ldb, ldc, layout, as_stream(stream));
}

}  // extern "C"
