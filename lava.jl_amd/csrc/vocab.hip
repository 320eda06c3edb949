// vocab.hip -- the tile-level vocabulary as kernels: one wavefront per tile.
//
// These entry points run the cooperative-matrix operations of
// src/vocabulary/coopmat.jl one tile at a time, exactly as a Lava kernel body
// strings them together, so that each operation's semantics (layouts, offsets,
// signedness, the lane -> (row, col) map, the reduce smear, RNE narrowing) can be
// checked element by element against the CPU oracle.
#include <hip/hip_runtime.h>

#include "lava_coopmat.hpp"
#include "lava_hip_internal.hpp"

namespace lava {

// ---- muladd on 16x16x16 tiles (docs/src/device.md:81-88) -------------------
template <typename TAB, typename TACC>
__global__ void __launch_bounds__(64) muladd_tile_kernel(const TAB* A, int64_t strideA, const TAB* B, int64_t strideB,
                                                         const TACC* C, int64_t strideC, TACC* D, int64_t strideD,
                                                         uint32_t layout, int64_t tile_step) {
    const int64_t t = blockIdx.x;
    const TAB* a_p = A + t * tile_step;
    const TAB* b_p = B + t * tile_step;
    const TACC* c_p = C + t * tile_step;
    TACC* d_p = D + t * tile_step;
    auto a = load<Frag<TAB, 16, 16, MatrixA>>(a_p, strideA, (layout & 1u) != 0);
    auto b = load<Frag<TAB, 16, 16, MatrixB>>(b_p, strideB, (layout & 2u) != 0);
    auto c = load<Frag<TACC, 16, 16, Accumulator>>(c_p, strideC, (layout & 4u) != 0);
    store(d_p, strideD, (layout & 8u) != 0, mma(a, b, c));
}

// Unsigned 8-bit: CDNA4's integer MFMA is signed, so each lane forms its four
// accumulator elements with v_dot4_u32_u8 over a row of A and a column of B.
__global__ void __launch_bounds__(64) muladd_tile_u8_kernel(const uint8_t* A, int64_t strideA, const uint8_t* B,
                                                            int64_t strideB, const uint32_t* C, int64_t strideC,
                                                            uint32_t* D, int64_t strideD, uint32_t layout,
                                                            int64_t tile_step) {
    const int64_t t = blockIdx.x;
    const uint8_t* a_p = A + t * tile_step;
    const uint8_t* b_p = B + t * tile_step;
    auto c = load<Frag<uint32_t, 16, 16, Accumulator>>(C + t * tile_step, strideC, (layout & 4u) != 0);
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = Layout<16, 16, Accumulator>::row(lane, j), n = Layout<16, 16, Accumulator>::col(lane, j);
        uint32_t s = c.v[j];
#pragma unroll
        for (int k = 0; k < 16; k += 4) {
            uint32_t x = 0, y = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                x |= (uint32_t)a_p[tile_index(r, k + q, strideA, (layout & 1u) != 0)] << (8 * q);
                y |= (uint32_t)b_p[tile_index(k + q, n, strideB, (layout & 2u) != 0)] << (8 * q);
            }
            s = __builtin_amdgcn_udot4(x, y, s, false);
        }
        c.v[j] = s;
    }
    store(D + t * tile_step, strideD, (layout & 8u) != 0, c);
}

// ---- per-element callbacks ---------------------------------------------------
// The known-answer callback of test/spirv/test_coopmat_perelement_inline.jl:20,
// which depends on both indices and is not symmetric under swapping them.
struct RowCol {
    __device__ float operator()(uint32_t row, uint32_t col, float e) const {
        // two roundings, as the Julia callback computes it (no fused multiply-add)
#pragma clang fp contract(off)
        return e * (float)(row + 1u) + (float)col;
    }
};

struct PairMax {
    __device__ float operator()(uint32_t row, uint32_t col, float x, float y) const {
        return fmaxf(x, y) + (float)row - (float)col;
    }
};

template <int T>
__global__ void __launch_bounds__(64) perelement_rowcol_kernel(const float* in, float* out) {
    const int64_t base = (int64_t)blockIdx.x * T * T;
    auto m = load<Frag<float, T, T, Accumulator>>(in + base, T, false);
    store(out + base, T, false, perelement(RowCol{}, m));
}

template <int T>
__global__ void __launch_bounds__(64) perelement_pair_kernel(const float* m_in, const float* o_in, float* out) {
    const int64_t base = (int64_t)blockIdx.x * T * T;
    auto m = load<Frag<float, T, T, Accumulator>>(m_in + base, T, false);
    auto o = load<Frag<float, T, T, Accumulator>>(o_in + base, T, false);
    store(out + base, T, false, perelement_m(PairMax{}, m, o));
}

// ---- reduce --------------------------------------------------------------------
struct CombineAdd {
    __device__ float operator()(float x, float y) const { return x + y; }
};
struct CombineMax {
    __device__ float operator()(float x, float y) const { return fmaxf(x, y); }
};
struct CombineMin {
    __device__ float operator()(float x, float y) const { return fminf(x, y); }
};

template <int T, uint32_t MASK, typename F>
__global__ void __launch_bounds__(64) reduce_kernel(const float* in, float* out) {
    const int64_t base = (int64_t)blockIdx.x * T * T;
    auto m = load<Frag<float, T, T, Accumulator>>(in + base, T, false);
    store(out + base, T, false, reduce<MASK>(F{}, m));
}

template <int T, uint32_t MASK>
static void launch_reduce(int combine, const float* in, float* out, int64_t n, hipStream_t s) {
    if (combine == LAVA_HIP_COMBINE_ADD)
        hipLaunchKernelGGL((reduce_kernel<T, MASK, CombineAdd>), dim3((unsigned)n), dim3(64), 0, s, in, out);
    else if (combine == LAVA_HIP_COMBINE_MAX)
        hipLaunchKernelGGL((reduce_kernel<T, MASK, CombineMax>), dim3((unsigned)n), dim3(64), 0, s, in, out);
    else
        hipLaunchKernelGGL((reduce_kernel<T, MASK, CombineMin>), dim3((unsigned)n), dim3(64), 0, s, in, out);
}

template <int T>
static void launch_reduce_mask(uint32_t mask, int combine, const float* in, float* out, int64_t n, hipStream_t s) {
    if (mask == 1u) launch_reduce<T, 1u>(combine, in, out, n, s);
    else if (mask == 2u) launch_reduce<T, 2u>(combine, in, out, n, s);
    else launch_reduce<T, 3u>(combine, in, out, n, s);
}

// ---- convert -------------------------------------------------------------------
template <typename To>
__global__ void __launch_bounds__(64) convert_kernel(const float* in, To* out) {
    const int64_t base = (int64_t)blockIdx.x * 256;
    auto m = load<Frag<float, 16, 16, Accumulator>>(in + base, 16, false);
    store(out + base, 16, false, convert<To>(m));
}

// ---- dot4x8 --------------------------------------------------------------------
__global__ void dot4x8_kernel(const uint32_t* a, const uint32_t* b, int32_t* y, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = dot4x8(a[i], b[i]);
}

static size_t dtype_size(int dt) {
    switch (dt) {
    case LAVA_HIP_F16:
    case LAVA_HIP_BF16: return 2;
    case LAVA_HIP_I8:
    case LAVA_HIP_U8: return 1;
    default: return 4;
    }
}

}  // namespace lava

using namespace lava;

extern "C" {

int lava_hip_coopmat_muladd_16x16x16(int ab_dtype, int acc_dtype, const void* A, int64_t offA, int64_t strideA,
                                     const void* B, int64_t offB, int64_t strideB, const void* C, int64_t offC,
                                     int64_t strideC, void* D, int64_t offD, int64_t strideD, uint32_t layout,
                                     int64_t ntiles, int64_t tile_step, void* stream) {
    const bool is_f16 = ab_dtype == LAVA_HIP_F16 && acc_dtype == LAVA_HIP_F32;
    const bool is_i8 = ab_dtype == LAVA_HIP_I8 && acc_dtype == LAVA_HIP_I32;
    const bool is_u8 = ab_dtype == LAVA_HIP_U8 && acc_dtype == LAVA_HIP_U32;
    LAVA_REQUIRE(is_f16 || is_i8 || is_u8, LAVA_HIP_ERR_UNSUPPORTED,
                 "coopmat_muladd_16x16x16: type pair (%d, %d) is not (F16,F32), (I8,I32) or (U8,U32)", ab_dtype,
                 acc_dtype);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_muladd_16x16x16: ntiles = %lld out of range",
             (long long)ntiles);
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(A && B && C && D, "coopmat_muladd_16x16x16: null pointer");
    LAVA_ARG(offA >= 1 && offB >= 1 && offC >= 1 && offD >= 1,
             "coopmat_muladd_16x16x16: offsets are 1-based and must be >= 1");
    LAVA_ARG(strideA >= 16 && strideB >= 16 && strideC >= 16 && strideD >= 16,
             "coopmat_muladd_16x16x16: strides must be >= 16");
    LAVA_ARG(tile_step >= 0, "coopmat_muladd_16x16x16: tile_step < 0");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const size_t sab = dtype_size(ab_dtype), sacc = dtype_size(acc_dtype);
    const char* a = static_cast<const char*>(A) + (offA - 1) * sab;
    const char* b = static_cast<const char*>(B) + (offB - 1) * sab;
    const char* c = static_cast<const char*>(C) + (offC - 1) * sacc;
    char* d = static_cast<char*>(D) + (offD - 1) * sacc;
    hipStream_t s = as_stream(stream);
    if (is_f16)
        hipLaunchKernelGGL((muladd_tile_kernel<lava::f16, float>), dim3((unsigned)ntiles), dim3(64), 0, s,
                           (const lava::f16*)a, strideA, (const lava::f16*)b, strideB, (const float*)c, strideC, (float*)d,
                           strideD, layout, tile_step);
    else if (is_i8)
        hipLaunchKernelGGL((muladd_tile_kernel<int8_t, int32_t>), dim3((unsigned)ntiles), dim3(64), 0, s,
                           (const int8_t*)a, strideA, (const int8_t*)b, strideB, (const int32_t*)c, strideC,
                           (int32_t*)d, strideD, layout, tile_step);
    else
        hipLaunchKernelGGL(muladd_tile_u8_kernel, dim3((unsigned)ntiles), dim3(64), 0, s, (const uint8_t*)a, strideA,
                           (const uint8_t*)b, strideB, (const uint32_t*)c, strideC, (uint32_t*)d, strideD, layout,
                           tile_step);
    LAVA_LAUNCH_CHECK("muladd_tile_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_perelement_rowcol(const float* in, float* out, int tile, int64_t ntiles, void* stream) {
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_perelement_rowcol: tile = %d is not 16 or 32", tile);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_perelement_rowcol: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(in && out, "coopmat_perelement_rowcol: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    if (tile == 16)
        hipLaunchKernelGGL(perelement_rowcol_kernel<16>, dim3((unsigned)ntiles), dim3(64), 0, as_stream(stream), in,
                           out);
    else
        hipLaunchKernelGGL(perelement_rowcol_kernel<32>, dim3((unsigned)ntiles), dim3(64), 0, as_stream(stream), in,
                           out);
    LAVA_LAUNCH_CHECK("perelement_rowcol_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_perelement_pair(const float* m, const float* o, float* out, int tile, int64_t ntiles,
                                     void* stream) {
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_perelement_pair: tile = %d is not 16 or 32", tile);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_perelement_pair: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(m && o && out, "coopmat_perelement_pair: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    if (tile == 16)
        hipLaunchKernelGGL(perelement_pair_kernel<16>, dim3((unsigned)ntiles), dim3(64), 0, as_stream(stream), m, o,
                           out);
    else
        hipLaunchKernelGGL(perelement_pair_kernel<32>, dim3((unsigned)ntiles), dim3(64), 0, as_stream(stream), m, o,
                           out);
    LAVA_LAUNCH_CHECK("perelement_pair_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_reduce(const float* in, float* out, int tile, uint32_t mask, int combine, int64_t ntiles,
                            void* stream) {
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_reduce: tile = %d is not 16 or 32", tile);
    LAVA_REQUIRE(mask != LAVA_HIP_REDUCE_TWO_BY_TWO, LAVA_HIP_ERR_UNSUPPORTED,
                 "coopmat_reduce: the TwoByTwo mask is not supported (the reference marks it unverified)");
    LAVA_ARG(mask >= 1u && mask <= 3u, "coopmat_reduce: mask %u is not Row, Column or RowAndColumn", mask);
    LAVA_ARG(combine >= LAVA_HIP_COMBINE_ADD && combine <= LAVA_HIP_COMBINE_MIN, "coopmat_reduce: combine %d unknown",
             combine);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_reduce: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(in && out, "coopmat_reduce: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    if (tile == 16) launch_reduce_mask<16>(mask, combine, in, out, ntiles, as_stream(stream));
    else launch_reduce_mask<32>(mask, combine, in, out, ntiles, as_stream(stream));
    LAVA_LAUNCH_CHECK("reduce_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_convert(const float* in, void* out, int out_dtype, int64_t n, void* stream) {
    LAVA_ARG(out_dtype == LAVA_HIP_F16 || out_dtype == LAVA_HIP_BF16, "coopmat_convert: dtype %d is not F16 or BF16",
             out_dtype);
    LAVA_ARG(n >= 0 && n % 256 == 0, "coopmat_convert: n = %lld is not a multiple of 256", (long long)n);
    LAVA_ARG(n / 256 <= 0x7fffffff, "coopmat_convert: n too large");
    if (n == 0) return LAVA_HIP_OK;
    LAVA_ARG(in && out, "coopmat_convert: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const unsigned g = (unsigned)(n / 256);
    if (out_dtype == LAVA_HIP_F16)
        hipLaunchKernelGGL(convert_kernel<lava::f16>, dim3(g), dim3(64), 0, as_stream(stream), in, (lava::f16*)out);
    else
        hipLaunchKernelGGL(convert_kernel<bf16>, dim3(g), dim3(64), 0, as_stream(stream), in, (bf16*)out);
    LAVA_LAUNCH_CHECK("convert_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_dot4x8(const uint32_t* a, const uint32_t* b, int32_t* y, int64_t n, void* stream) {
    LAVA_ARG(n >= 0, "dot4x8: n < 0");
    if (n == 0) return LAVA_HIP_OK;
    LAVA_ARG(a && b && y, "dot4x8: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    int64_t g = (n + 255) / 256;
    if (g > 8192) g = 8192;
    hipLaunchKernelGGL(dot4x8_kernel, dim3((unsigned)g), dim3(256), 0, as_stream(stream), a, b, y, n);
    LAVA_LAUNCH_CHECK("dot4x8_kernel");
    return LAVA_HIP_OK;
}

}  // extern "C"
