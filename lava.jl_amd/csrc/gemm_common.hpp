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

// One 32x32 MFMA step with 16-byte-per-lane operands: 8 x fp16 / 8 x bf16
// (32x32x16) or 16 x int8 (32x32x32).  Operand lane l holds row (or column) l % 32
// and k-slots 8 (l / 32) + [0, 8) (16-bit) or 16 (l / 32) + [0, 16) (int8); the
// accumulator lane holds column l % 32, rows 8 (j / 4) + 4 (l / 32) + j % 4.
template <typename T>
struct Mfma32;

template <>
struct Mfma32<f16> {
    typedef f32x16 acc_t;
    __device__ static acc_t run(uint4 a, uint4 b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    }
};

template <>
struct Mfma32<bf16> {
    typedef f32x16 acc_t;
    __device__ static acc_t run(uint4 a, uint4 b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    }
};

template <>
struct Mfma32<int8_t> {
    typedef i32x16 acc_t;
    __device__ static acc_t run(uint4 a, uint4 b, acc_t c) {
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0,
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

}  // namespace lava
