// fill.hip -- the seeded input generator, on the device.
//
// Definition (identical to the CPU oracle's, element by element):
//   draw(seed, i)  = splitmix64 finaliser of seed*0xD1B54A32D192ED03 + (i+1)*0x9E3779B97F4A7C15
//   uniform[a,b]   = fl32(a + (b-a) * (draw >> 40) * 2^-24), computed in binary64
//   normal(0,1)    = fl32(sqrt(-2 ln u1) cos(2 pi u2)), u1/u2 = (hi/lo 32 bits + 0.5) 2^-32
//   int8 [-128,127]= top byte of the draw; int8 [-127,127] = (draw >> 32) mod 255 - 127
// then RNE to the storage type.
#include <hip/hip_runtime.h>

#include "lava_coopmat.hpp"
#include "lava_hip_internal.hpp"

namespace lava {

__device__ __forceinline__ uint64_t rng_u64(uint64_t seed, uint64_t i) {
    uint64_t z = seed * 0xD1B54A32D192ED03ull + (i + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <typename T>
__device__ __forceinline__ void put(void* dst, int64_t i, float v) {
    static_cast<T*>(dst)[i] = narrow<T>(v);
}

template <typename T>
__global__ void fill_uniform_kernel(void* dst, int64_t n, uint64_t seed, double a, double span) {
    // the definition rounds the product and the sum separately: no fma contraction
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t k = rng_u64(seed, (uint64_t)i) >> 40;
        const double t = span * ((double)k * 5.9604644775390625e-08);
        put<T>(dst, i, (float)(a + t));
    }
}

template <typename T>
__global__ void fill_normal_kernel(void* dst, int64_t n, uint64_t seed) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t z = rng_u64(seed, (uint64_t)i);
        const double u1 = ((double)(z >> 32) + 0.5) * 2.3283064365386963e-10;
        const double u2 = ((double)(z & 0xffffffffull) + 0.5) * 2.3283064365386963e-10;
        const double r = sqrt(-2.0 * log(u1));
        put<T>(dst, i, (float)(r * cos(6.283185307179586 * u2)));
    }
}

__global__ void fill_i8_kernel(int8_t* dst, int64_t n, uint64_t seed, int symmetric) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t z = rng_u64(seed, (uint64_t)i);
        dst[i] = symmetric ? (int8_t)((int)((z >> 32) % 255u) - 127) : (int8_t)(uint8_t)(z >> 56);
    }
}

static unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    if (g > 8192) g = 8192;
    if (g < 1) g = 1;
    return (unsigned)g;
}

}  // namespace lava

using namespace lava;

extern "C" {

int lava_hip_fill_uniform(void* dst, int dtype, int64_t n, uint64_t seed, double a, double b, void* stream) {
    LAVA_ARG(n >= 0, "fill_uniform: n = %lld < 0", (long long)n);
    if (n == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr, "fill_uniform: null destination");
    LAVA_ARG(dtype == LAVA_HIP_F16 || dtype == LAVA_HIP_BF16 || dtype == LAVA_HIP_F32,
             "fill_uniform: dtype %d is not F16, BF16 or F32", dtype);
    hipStream_t s = as_stream(stream);
    const double span = b - a;
    if (dtype == LAVA_HIP_F16)
        hipLaunchKernelGGL(fill_uniform_kernel<f16>, dim3(grid_for(n)), dim3(256), 0, s, dst, n, seed, a, span);
    else if (dtype == LAVA_HIP_BF16)
        hipLaunchKernelGGL(fill_uniform_kernel<bf16>, dim3(grid_for(n)), dim3(256), 0, s, dst, n, seed, a, span);
    else
        hipLaunchKernelGGL(fill_uniform_kernel<float>, dim3(grid_for(n)), dim3(256), 0, s, dst, n, seed, a, span);
    LAVA_LAUNCH_CHECK("fill_uniform_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_fill_normal(void* dst, int dtype, int64_t n, uint64_t seed, void* stream) {
    LAVA_ARG(n >= 0, "fill_normal: n = %lld < 0", (long long)n);
    if (n == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr, "fill_normal: null destination");
    LAVA_ARG(dtype == LAVA_HIP_F16 || dtype == LAVA_HIP_BF16 || dtype == LAVA_HIP_F32,
             "fill_normal: dtype %d is not F16, BF16 or F32", dtype);
    hipStream_t s = as_stream(stream);
    if (dtype == LAVA_HIP_F16)
        hipLaunchKernelGGL(fill_normal_kernel<f16>, dim3(grid_for(n)), dim3(256), 0, s, dst, n, seed);
    else if (dtype == LAVA_HIP_BF16)
        hipLaunchKernelGGL(fill_normal_kernel<bf16>, dim3(grid_for(n)), dim3(256), 0, s, dst, n, seed);
    else
        hipLaunchKernelGGL(fill_normal_kernel<float>, dim3(grid_for(n)), dim3(256), 0, s, dst, n, seed);
    LAVA_LAUNCH_CHECK("fill_normal_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_fill_i8(void* dst, int64_t n, uint64_t seed, int symmetric, void* stream) {
    LAVA_ARG(n >= 0, "fill_i8: n = %lld < 0", (long long)n);
    if (n == 0) return LAVA_HIP_OK;
    LAVA_ARG(dst != nullptr, "fill_i8: null destination");
    hipLaunchKernelGGL(fill_i8_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
                       static_cast<int8_t*>(dst), n, seed, symmetric);
    LAVA_LAUNCH_CHECK("fill_i8_kernel");
    return LAVA_HIP_OK;
}

}  // extern "C"
