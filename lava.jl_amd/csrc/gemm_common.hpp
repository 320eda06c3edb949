// gemm_common.hpp -- pieces shared by the GEMM kernels.
#pragma once
#include <hip/hip_runtime.h>

#include "lava_coopmat.hpp"

namespace lava {

// One 16x16 MFMA step whose A and B operands are 16 bytes per lane:
// 8 x fp16 / 8 x bf16 (16x16x32) or 16 x int8 (16x16x64).  The accumulator is
// 4 x fp32 or 4 x int32; lane holds column lane % 16, rows 4 * (lane / 16) + j.
template <typename T>
struct Mfma16;

template <>
struct Mfma16<f16> {
    typedef f32x4 acc_t;
    typedef float acc_elem;
    static constexpr int k = 32;
    __device__ static acc_t run(uint4 a, uint4 b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    }
};

template <>
struct Mfma16<bf16> {
    typedef f32x4 acc_t;
    typedef float acc_elem;
    static constexpr int k = 32;
    __device__ static acc_t run(uint4 a, uint4 b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    }
};

template <>
struct Mfma16<int8_t> {
    typedef i32x4 acc_t;
    typedef int32_t acc_elem;
    static constexpr int k = 64;
    __device__ static acc_t run(uint4 a, uint4 b, acc_t c) {
        return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0,
                                                     0, 0);
    }
};

// MI355X places workgroup b on XCD b % 8 and each XCD has its own L2.  Renumber
// so that the tiles one XCD runs at the same time form a compact block of C
// (rows of A and columns of B that the XCD's L2 then shares):
//   1. consecutive logical ids per XCD: t = (b % 8) * (n / 8) + b / 8;
//   2. grouped order: `group_m` tile rows at a time, tile row fastest.
// Falls back to the identity when n is not a multiple of 8.
__device__ __forceinline__ void xcd_tile(int b, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int n = tiles_m * tiles_n;
    int t = b;
    if ((n & 7) == 0) t = (b & 7) * (n >> 3) + (b >> 3);
    const int per_group = group_m * tiles_n;
    const int g = t / per_group;
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int r = t - g * per_group;
    tm = first_m + r % gm;
    tn = r / gm;
}

// ---- fused GEMM epilogue: D = act(A B + (bias + residual)), then narrowed to D's type.
// Lava starts the accumulator from bias + residual (`accinit`: a stride-0
// accumulator load of the bias plus the residual at its leading dimension, summed
// with coopmat_add, src/device/coopmat_intrinsics.jl:435-464), applies elementwise
// epilogues through getcomp / setcomp (:322-400) and narrows with coopmat_convert
// (RNE, src/compiler/spirv/coopmat.jl:783-824).  Here the same terms are added to the
// finished accumulator in the store: the same sum, in another fp32 order.
enum EpiAct : int { EPI_NONE = 0, EPI_RELU = 1, EPI_GELU_TANH = 2, EPI_GELU_ERF = 3 };

struct Epilogue {
    const float* bias = nullptr;       // nullptr, or one value per row (per column if bias_on_cols) of D
    const float* residual = nullptr;   // nullptr, or a matrix laid out like D (row-major here) with ldr
    int64_t ldr = 0;
    int bias_on_cols = 0;              // D was transposed to row-major: the bias then runs along columns
    int act = EPI_NONE;
    int vec4 = 0;                      // bias and residual 16-byte aligned, ldr % 4 == 0: 4 columns per load
};

// The extents a RAGGED TN launch checks against: M, N, K in bytes, and whether C rows
// take 4-element vector stores (ldc % 4 == 0, C aligned to 4 elements).
struct TnBounds {
    int64_t m = 0, n = 0;
    int kb = 0;
    int cvec = 0;
};

// Inline elementary functions (a library call here would have to save the 256
// accumulator registers that are still live around the epilogue):
// e^x through v_exp_f32; tanh(u) = sign(u) (1 - e^{-2|u|}) / (1 + e^{-2|u|});
// erf by Abramowitz & Stegun, Handbook of Mathematical Functions, 7.1.26
// (|error| <= 1.5e-7 over the real line).
__device__ __forceinline__ float epi_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
// The quotients use v_rcp_f32 (1 ulp) instead of the IEEE division sequence: a
// tenth of the instructions, and far inside the GEMM's 1e-3 tolerance.
__device__ __forceinline__ float epi_tanh(float u) {
    const float e = epi_exp(-2.f * fabsf(u));
    return copysignf((1.f - e) * __builtin_amdgcn_rcpf(1.f + e), u);
}
__device__ __forceinline__ float epi_erf(float x) {
    const float ax = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(1.f + 0.3275911f * ax);
    const float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
    return copysignf(1.f - p * epi_exp(-ax * ax), x);
}

// The activation as a compile-time constant: a store loop instantiated per activation
// carries no per-element branch.
template <int ACT>
__device__ __forceinline__ float epi_act_c(float v) {
    if constexpr (ACT == EPI_RELU) {
        return v > 0.f ? v : 0.f;
    } else if constexpr (ACT == EPI_GELU_TANH) {
        // 0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3)))
        const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
        return 0.5f * v * (1.f + epi_tanh(u));
    } else if constexpr (ACT == EPI_GELU_ERF) {
        return 0.5f * v * (1.f + epi_erf(v * 0.7071067811865476f));   // 0.5 x (1 + erf(x / sqrt 2))
    } else {
        return v;
    }
}

__device__ __forceinline__ float epi_act(int act, float v) {
    switch (act) {
    case EPI_RELU: return epi_act_c<EPI_RELU>(v);
    case EPI_GELU_TANH: return epi_act_c<EPI_GELU_TANH>(v);
    case EPI_GELU_ERF: return epi_act_c<EPI_GELU_ERF>(v);
    default: return v;
    }
}

// The finished accumulator value of D[m][n] (row-major frame of the kernel) through the epilogue.
__device__ __forceinline__ float epi_apply(const Epilogue& e, int64_t m, int64_t n, float acc) {
    float init = 0.f;
    if (e.bias) init = e.bias[e.bias_on_cols ? n : m];
    if (e.residual) init += e.residual[m * e.ldr + n];
    return epi_act(e.act, acc + init);
}

}  // namespace lava
