// vocab.hip -- the tile-level vocabulary as kernels: one wavefront per tile.
//
// These entry points run the cooperative-matrix operations of
// src/vocabulary/coopmat.jl one tile at a time, exactly as a Lava kernel body
// strings them together, so that each operation's semantics (layouts, offsets,
// signedness, the lane -> (row, col) map, the reduce smear, RNE narrowing) can be
// checked element by element against the CPU oracle.
#include <hip/hip_runtime.h>

#include "gemm_common.hpp"
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

// fp32 and fp64 operands: a 16x16x16 tile is four 16x16x4 MFMAs.  Lane (r, g) = (lane % 16,
// lane / 16) supplies A[r][4 s + g] and B[4 s + g][r] to step s.  Its accumulator element i is
// C[4 g + i][r] for fp32 (the layout of the other 16x16 MFMAs) but C[g + 4 i][r] for fp64 (the
// 16x16x4 fp64 MFMA interleaves its rows; measured, and pinned by the identity-product tests).
template <typename T>
__global__ void __launch_bounds__(64) muladd_tile_wide_kernel(const T* A, int64_t strideA, const T* B,
                                                              int64_t strideB, const T* C, int64_t strideC, T* D,
                                                              int64_t strideD, uint32_t layout, int64_t tile_step) {
    typedef T v4 __attribute__((ext_vector_type(4)));
    const int64_t t = blockIdx.x;
    const T* a_p = A + t * tile_step;
    const T* b_p = B + t * tile_step;
    const T* c_p = C + t * tile_step;
    T* d_p = D + t * tile_step;
    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
    const bool arow = layout & 1u, brow = layout & 2u, crow = layout & 4u, drow = layout & 8u;
    v4 acc;
    auto row = [&](int i) { return sizeof(T) == 8 ? g + 4 * i : 4 * g + i; };
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = c_p[tile_index(row(i), r, strideC, crow)];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        const T a = a_p[tile_index(r, 4 * st + g, strideA, arow)];
        const T b = b_p[tile_index(4 * st + g, r, strideB, brow)];
        if constexpr (sizeof(T) == 8)
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc, 0, 0, 0);
        else
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) d_p[tile_index(row(i), r, strideD, drow)] = acc[i];
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

// reduce into a destination of another extent: one wavefront per tile, column-major tiles in
// memory like the same-shape form
template <int T, uint32_t MASK, int RD, int CD, typename F>
__global__ void __launch_bounds__(64) reduce_into_kernel(const float* in, float* out) {
    __shared__ float lds[T * T];
    auto m = load<Frag<float, T, T, Accumulator>>(in + (int64_t)blockIdx.x * T * T, T, false);
    const auto d = reduce_into<MASK, RD, CD>(F{}, m, lds);
    store(out + (int64_t)blockIdx.x * RD * CD, RD, false, d);
}

template <int T, uint32_t MASK, int RD, int CD>
static void launch_reduce_into(int combine, const float* in, float* out, int64_t n, hipStream_t s) {
    if (combine == LAVA_HIP_COMBINE_ADD)
        hipLaunchKernelGGL((reduce_into_kernel<T, MASK, RD, CD, CombineAdd>), dim3((unsigned)n), dim3(64), 0, s, in, out);
    else if (combine == LAVA_HIP_COMBINE_MAX)
        hipLaunchKernelGGL((reduce_into_kernel<T, MASK, RD, CD, CombineMax>), dim3((unsigned)n), dim3(64), 0, s, in, out);
    else
        hipLaunchKernelGGL((reduce_into_kernel<T, MASK, RD, CD, CombineMin>), dim3((unsigned)n), dim3(64), 0, s, in, out);
}

// The destination extents the entry instantiates: 16, 32 or 64 along a free axis.
template <int T, uint32_t MASK, int RD>
static bool reduce_into_cols(int cd, int combine, const float* in, float* out, int64_t n, hipStream_t s) {
    switch (cd) {
    case 16: launch_reduce_into<T, MASK, RD, 16>(combine, in, out, n, s); return true;
    case 32: launch_reduce_into<T, MASK, RD, 32>(combine, in, out, n, s); return true;
    case 64: launch_reduce_into<T, MASK, RD, 64>(combine, in, out, n, s); return true;
    default: return false;
    }
}

template <int T>
static bool launch_reduce_into_mask(uint32_t mask, int rd, int cd, int combine, const float* in, float* out, int64_t n,
                                    hipStream_t s) {
    if (mask == 4u) {
        if (rd != T / 2 || cd != T / 2) return false;
        launch_reduce_into<T, 4u, T / 2, T / 2>(combine, in, out, n, s);
        return true;
    }
    if (mask == 1u) return rd == T && reduce_into_cols<T, 1u, T>(cd, combine, in, out, n, s);
    if (mask == 2u) {
        if (cd != T) return false;
        switch (rd) {
        case 16: launch_reduce_into<T, 2u, 16, T>(combine, in, out, n, s); return true;
        case 32: launch_reduce_into<T, 2u, 32, T>(combine, in, out, n, s); return true;
        case 64: launch_reduce_into<T, 2u, 64, T>(combine, in, out, n, s); return true;
        default: return false;
        }
    }
    switch (rd) {
    case 16: return reduce_into_cols<T, 3u, 16>(cd, combine, in, out, n, s);
    case 32: return reduce_into_cols<T, 3u, 32>(cd, combine, in, out, n, s);
    case 64: return reduce_into_cols<T, 3u, 64>(cd, combine, in, out, n, s);
    default: return false;
    }
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


// ---- convert with a change of use (src/device/coopmat_intrinsics.jl:222-247) ----------
// The fp32 Accumulator tile becomes a To tile of use UTo and is stored through UTo's
// lane map, so the stored matrix equals the narrowed input exactly when every element
// reached the lane and slot UTo assigns to it.
template <int T, typename To, Use UTo>
__global__ void __launch_bounds__(64) convert_use_kernel(const float* in, To* out) {
    __shared__ To scratch[T * T];
    const int64_t base = (int64_t)blockIdx.x * T * T;
    auto m = load<Frag<float, T, T, Accumulator>>(in + base, T, false);
    store(out + base, T, false, convert<To, UTo>(m, scratch));
}

// Attention's second product: P (fp32 Accumulator) -> fp16 MatrixA, times V (MatrixB).
__global__ void __launch_bounds__(64) convert_use_muladd_kernel(const float* P, const f16* V, float* D) {
    __shared__ f16 scratch[256];
    const int64_t base = (int64_t)blockIdx.x * 256;
    auto p = load<Frag<float, 16, 16, Accumulator>>(P + base, 16, false);
    auto pa = convert<f16, MatrixA>(p, scratch);
    auto v = load<Frag<f16, 16, 16, MatrixB>>(V + base, 16, false);
    store(D + base, 16, false, mma(pa, v, zero<Frag<float, 16, 16, Accumulator>>()));
}

// ---- coopmat_mul / coopmat_add (src/device/coopmat_intrinsics.jl:402-464) ------------
// Operands are Accumulator loads; a stride of 0 makes every column (column-major) or
// every row (row-major) read the same vector.
template <int T, int OP>
__global__ void __launch_bounds__(64) elementwise_kernel(const float* A, int64_t sa, const float* B, int64_t sb,
                                                         float* D, int64_t sd, uint32_t layout, int64_t step) {
    const int64_t t = blockIdx.x;
    auto a = load<Frag<float, T, T, Accumulator>>(A + t * step, sa, (layout & 1u) != 0);
    auto b = load<Frag<float, T, T, Accumulator>>(B + t * step, sb, (layout & 2u) != 0);
    store(D + t * step, sd, (layout & 4u) != 0, OP == LAVA_HIP_ELEMENTWISE_MUL ? mul(a, b) : add(a, b));
}

// `accinit`: the accumulator starts from bias (stride-0 load, one value per row) plus the
// residual (its own leading dimension), summed with coopmat_add, then muladd.
__global__ void __launch_bounds__(64) accinit_muladd_kernel(const f16* A, const f16* B, const float* bias,
                                                            const float* R, int64_t ldr, float* D, int64_t ldd) {
    const int64_t t = blockIdx.x;
    auto a = load<Frag<f16, 16, 16, MatrixA>>(A + t * 256, 16, false);
    auto b = load<Frag<f16, 16, 16, MatrixB>>(B + t * 256, 16, false);
    auto bias0 = load<Frag<float, 16, 16, Accumulator>>(bias + t * 16, 0, false);
    auto res = load<Frag<float, 16, 16, Accumulator>>(R + t * 16 * ldr, ldr, false);
    store(D + t * 16 * ldd, ldd, false, mma(a, b, add(bias0, res)));
}

// ---- the portable elementwise epilogue: for i in 0:length-1, setcomp(m, i, f(getcomp(m, i)))
// (src/device/coopmat_intrinsics.jl:322-400) -----------------------------------------------
template <int T, int ACT>
__global__ void __launch_bounds__(64) foreach_act_kernel(const float* in, float* out, int32_t* len_out) {
    const int64_t base = (int64_t)blockIdx.x * T * T;
    auto m = load<Frag<float, T, T, Accumulator>>(in + base, T, false);
    const int n = length(m);
    for (int i = 0; i < n; ++i) m = setcomp(m, i, epi_act_c<ACT>(getcomp(m, i)));
    store(out + base, T, false, m);
    if (blockIdx.x == 0 && threadIdx.x == 0) *len_out = n;
}

// ---- coopmat_perelement(f, m, extras...) with a pointer and an offset in extras
// (src/device/coopmat_intrinsics.jl:569-572): the W8A16 dequant e * s[base + col] and
// attention's rescale e * cs[base + row] ------------------------------------------------------
struct ScaleByColumn {
    __device__ float operator()(uint32_t, uint32_t col, float e, const f16* s, uint32_t base) const {
        return e * (float)s[base + col];
    }
};
struct ScaleByRow {
    __device__ float operator()(uint32_t row, uint32_t, float e, const float* cs, uint32_t base) const {
        return e * cs[base + row];
    }
};

template <int T, bool BY_ROW>
__global__ void __launch_bounds__(64) perelement_scale_kernel(const float* in, float* out, const void* factors,
                                                              uint32_t base) {
    const int64_t off = (int64_t)blockIdx.x * T * T;
    auto m = load<Frag<float, T, T, Accumulator>>(in + off, T, false);
    const uint32_t tb = base + (uint32_t)blockIdx.x * T;
    if constexpr (BY_ROW)
        m = perelement(ScaleByRow{}, m, static_cast<const float*>(factors), tb);
    else
        m = perelement(ScaleByColumn{}, m, static_cast<const f16*>(factors), tb);
    store(out + off, T, false, m);
}

// ---- workgroup-scope matrices -----------------------------------------------------------
// A workgroup-scope matrix at NT invocations is held by its NT / 64 wavefronts, arranged
// WM x WN, wavefront (wm, wn) holding the 16 x 16 tiles (i, j) with i % WM == wm and
// j % WN == wn; K advances in steps of the 16x16x16 instruction.  Its (M, N, K) must be
// multiples of (16 WM, 16 WN, 16): the rows of the `wggran` table (caps.jl:122-145).
struct WgShape {
    int nt, wm, wn;
};
constexpr WgShape kWgShapes[] = {{64, 1, 1}, {128, 2, 1}, {256, 2, 2}, {512, 4, 2}, {1024, 4, 4}};

template <int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64) workgroup_gemm_kernel(const f16* A, const f16* B, float* C, int M,
                                                                      int N, int K, int64_t lda, int64_t ldb,
                                                                      int64_t ldc, uint32_t layout) {
    const int w = threadIdx.x >> 6, wm = w / WN, wn = w % WN;
    const bool arow = layout & 1u, brow = layout & 2u, crow = layout & 4u;
    for (int i = wm; i < M / 16; i += WM)
        for (int j = wn; j < N / 16; j += WN) {
            auto acc = zero<Frag<float, 16, 16, Accumulator>>();
            for (int k = 0; k < K / 16; ++k) {
                auto a = load<Frag<f16, 16, 16, MatrixA>>(A + tile_index(16 * i, 16 * k, lda, arow), lda, arow);
                auto b = load<Frag<f16, 16, 16, MatrixB>>(B + tile_index(16 * k, 16 * j, ldb, brow), ldb, brow);
                acc = mma(a, b, acc);
            }
            store(C + tile_index(16 * i, 16 * j, ldc, crow), ldc, crow, acc);
        }
}

static size_t dtype_size(int dt) {
    switch (dt) {
    case LAVA_HIP_F16:
    case LAVA_HIP_BF16: return 2;
    case LAVA_HIP_I8:
    case LAVA_HIP_U8: return 1;
    case LAVA_HIP_F64: return 8;
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
    const bool is_f32 = ab_dtype == LAVA_HIP_F32 && acc_dtype == LAVA_HIP_F32;
    const bool is_f64 = ab_dtype == LAVA_HIP_F64 && acc_dtype == LAVA_HIP_F64;
    LAVA_REQUIRE(is_f16 || is_i8 || is_u8 || is_f32 || is_f64, LAVA_HIP_ERR_UNSUPPORTED,
                 "coopmat_muladd_16x16x16: type pair (%d, %d) is not (F16,F32), (I8,I32), (U8,U32), (F32,F32) or "
                 "(F64,F64)", ab_dtype, acc_dtype);
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
    else if (is_f32)
        hipLaunchKernelGGL(muladd_tile_wide_kernel<float>, dim3((unsigned)ntiles), dim3(64), 0, s, (const float*)a,
                           strideA, (const float*)b, strideB, (const float*)c, strideC, (float*)d, strideD, layout,
                           tile_step);
    else if (is_f64)
        hipLaunchKernelGGL(muladd_tile_wide_kernel<double>, dim3((unsigned)ntiles), dim3(64), 0, s, (const double*)a,
                           strideA, (const double*)b, strideB, (const double*)c, strideC, (double*)d, strideD, layout,
                           tile_step);
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
                 "coopmat_reduce: a TwoByTwo reduce halves both extents; use lava_hip_coopmat_reduce_into");
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

int lava_hip_coopmat_reduce_into(const float* in, float* out, int tile, int dst_rows, int dst_cols, uint32_t mask,
                                 int combine, int64_t ntiles, void* stream) {
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_reduce_into: tile = %d is not 16 or 32", tile);
    LAVA_ARG(mask >= 1u && mask <= 4u, "coopmat_reduce_into: mask %u is not Row, Column, RowAndColumn or TwoByTwo",
             mask);
    LAVA_ARG(combine >= LAVA_HIP_COMBINE_ADD && combine <= LAVA_HIP_COMBINE_MIN,
             "coopmat_reduce_into: combine %d unknown", combine);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_reduce_into: ntiles out of range");
    const bool shape_ok =
        mask == 4u ? dst_rows == tile / 2 && dst_cols == tile / 2
                   : (mask == 1u ? dst_rows == tile : (dst_rows == 16 || dst_rows == 32 || dst_rows == 64)) &&
                         (mask == 2u ? dst_cols == tile : (dst_cols == 16 || dst_cols == 32 || dst_cols == 64));
    LAVA_ARG(shape_ok,
             "coopmat_reduce_into: destination %d x %d does not fit mask %u on %d x %d tiles (Row keeps the rows, "
             "Column the columns, a free extent is 16, 32 or 64; TwoByTwo halves both)",
             dst_rows, dst_cols, mask, tile, tile);
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(in && out, "coopmat_reduce_into: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const bool ok = tile == 16
                        ? launch_reduce_into_mask<16>(mask, dst_rows, dst_cols, combine, in, out, ntiles, as_stream(stream))
                        : launch_reduce_into_mask<32>(mask, dst_rows, dst_cols, combine, in, out, ntiles, as_stream(stream));
    LAVA_REQUIRE(ok, LAVA_HIP_ERR_UNSUPPORTED, "coopmat_reduce_into: no instance for this shape");
    LAVA_LAUNCH_CHECK("reduce_into_kernel");
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

int lava_hip_coopmat_convert_use(const float* in, void* out, int out_dtype, int tile, int use, int64_t ntiles,
                                 void* stream) {
    LAVA_ARG(out_dtype == LAVA_HIP_F16 || out_dtype == LAVA_HIP_BF16, "coopmat_convert_use: dtype %d is not F16 or BF16",
             out_dtype);
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_convert_use: tile = %d is not 16 or 32", tile);
    LAVA_ARG(use == LAVA_HIP_USE_MATRIX_A || use == LAVA_HIP_USE_MATRIX_B || use == LAVA_HIP_USE_ACCUMULATOR,
             "coopmat_convert_use: use %d is not MatrixA, MatrixB or Accumulator", use);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_convert_use: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(in && out, "coopmat_convert_use: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const dim3 g((unsigned)ntiles);
    hipStream_t s = as_stream(stream);
#define LAVA_CONVERT_USE(T, TO)                                                                                     \
    do {                                                                                                            \
        if (use == LAVA_HIP_USE_MATRIX_A)                                                                           \
            hipLaunchKernelGGL((convert_use_kernel<T, TO, MatrixA>), g, dim3(64), 0, s, in, (TO*)out);             \
        else if (use == LAVA_HIP_USE_MATRIX_B)                                                                      \
            hipLaunchKernelGGL((convert_use_kernel<T, TO, MatrixB>), g, dim3(64), 0, s, in, (TO*)out);             \
        else                                                                                                        \
            hipLaunchKernelGGL((convert_use_kernel<T, TO, Accumulator>), g, dim3(64), 0, s, in, (TO*)out);         \
    } while (0)
    if (tile == 16 && out_dtype == LAVA_HIP_F16) LAVA_CONVERT_USE(16, lava::f16);
    else if (tile == 16) LAVA_CONVERT_USE(16, bf16);
    else if (out_dtype == LAVA_HIP_F16) LAVA_CONVERT_USE(32, lava::f16);
    else LAVA_CONVERT_USE(32, bf16);
#undef LAVA_CONVERT_USE
    LAVA_LAUNCH_CHECK("convert_use_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_convert_use_muladd_16x16x16(const float* P, const void* V, float* D, int64_t ntiles,
                                                 void* stream) {
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_convert_use_muladd: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(P && V && D, "coopmat_convert_use_muladd: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipLaunchKernelGGL(convert_use_muladd_kernel, dim3((unsigned)ntiles), dim3(64), 0, as_stream(stream), P,
                       (const lava::f16*)V, D);
    LAVA_LAUNCH_CHECK("convert_use_muladd_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_elementwise(int op, int tile, const float* A, int64_t strideA, const float* B, int64_t strideB,
                                 float* D, int64_t strideD, uint32_t layout, int64_t ntiles, int64_t tile_step,
                                 void* stream) {
    LAVA_ARG(op == LAVA_HIP_ELEMENTWISE_MUL || op == LAVA_HIP_ELEMENTWISE_ADD, "coopmat_elementwise: op %d unknown", op);
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_elementwise: tile = %d is not 16 or 32", tile);
    LAVA_ARG(layout <= 7u, "coopmat_elementwise: layout %u has bits beyond A, B, D row-major", layout);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_elementwise: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(A && B && D, "coopmat_elementwise: null pointer");
    LAVA_ARG(strideA >= 0 && strideB >= 0 && strideD >= tile && tile_step >= 0,
             "coopmat_elementwise: operand strides must be >= 0 (0 broadcasts), D's >= tile, tile_step >= 0");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const dim3 g((unsigned)ntiles);
    hipStream_t s = as_stream(stream);
    if (tile == 16 && op == LAVA_HIP_ELEMENTWISE_MUL)
        hipLaunchKernelGGL((elementwise_kernel<16, LAVA_HIP_ELEMENTWISE_MUL>), g, dim3(64), 0, s, A, strideA, B,
                           strideB, D, strideD, layout, tile_step);
    else if (tile == 16)
        hipLaunchKernelGGL((elementwise_kernel<16, LAVA_HIP_ELEMENTWISE_ADD>), g, dim3(64), 0, s, A, strideA, B,
                           strideB, D, strideD, layout, tile_step);
    else if (op == LAVA_HIP_ELEMENTWISE_MUL)
        hipLaunchKernelGGL((elementwise_kernel<32, LAVA_HIP_ELEMENTWISE_MUL>), g, dim3(64), 0, s, A, strideA, B,
                           strideB, D, strideD, layout, tile_step);
    else
        hipLaunchKernelGGL((elementwise_kernel<32, LAVA_HIP_ELEMENTWISE_ADD>), g, dim3(64), 0, s, A, strideA, B,
                           strideB, D, strideD, layout, tile_step);
    LAVA_LAUNCH_CHECK("elementwise_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_accinit_muladd_16x16x16(const void* A, const void* B, const float* bias, const float* residual,
                                             int64_t ldr, float* D, int64_t ldd, int64_t ntiles, void* stream) {
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_accinit_muladd: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(A && B && bias && residual && D, "coopmat_accinit_muladd: null pointer");
    LAVA_ARG(ldr >= 16 && ldd >= 16, "coopmat_accinit_muladd: ldr and ldd must be >= 16");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipLaunchKernelGGL(accinit_muladd_kernel, dim3((unsigned)ntiles), dim3(64), 0, as_stream(stream),
                       (const lava::f16*)A, (const lava::f16*)B, bias, residual, ldr, D, ldd);
    LAVA_LAUNCH_CHECK("accinit_muladd_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_foreach_act(const float* in, float* out, int tile, int act, int64_t ntiles, int32_t* length_out,
                                 void* stream) {
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_foreach_act: tile = %d is not 16 or 32", tile);
    LAVA_ARG(act >= LAVA_HIP_ACT_NONE && act <= LAVA_HIP_ACT_GELU_ERF, "coopmat_foreach_act: act %d unknown", act);
    LAVA_ARG(ntiles >= 1 && ntiles <= 0x7fffffff, "coopmat_foreach_act: ntiles out of range (>= 1)");
    LAVA_ARG(in && out && length_out, "coopmat_foreach_act: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const dim3 g((unsigned)ntiles);
    hipStream_t s = as_stream(stream);
#define LAVA_FOREACH(T)                                                                                          \
    do {                                                                                                         \
        switch (act) {                                                                                           \
        case LAVA_HIP_ACT_RELU:                                                                                  \
            hipLaunchKernelGGL((foreach_act_kernel<T, EPI_RELU>), g, dim3(64), 0, s, in, out, length_out);       \
            break;                                                                                               \
        case LAVA_HIP_ACT_GELU_TANH:                                                                             \
            hipLaunchKernelGGL((foreach_act_kernel<T, EPI_GELU_TANH>), g, dim3(64), 0, s, in, out, length_out);  \
            break;                                                                                               \
        case LAVA_HIP_ACT_GELU_ERF:                                                                              \
            hipLaunchKernelGGL((foreach_act_kernel<T, EPI_GELU_ERF>), g, dim3(64), 0, s, in, out, length_out);   \
            break;                                                                                               \
        default: hipLaunchKernelGGL((foreach_act_kernel<T, EPI_NONE>), g, dim3(64), 0, s, in, out, length_out); \
        }                                                                                                        \
    } while (0)
    if (tile == 16) LAVA_FOREACH(16);
    else LAVA_FOREACH(32);
#undef LAVA_FOREACH
    LAVA_LAUNCH_CHECK("foreach_act_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_length(int dtype, int rows, int cols, int use, int32_t* length_out) {
    LAVA_ARG(length_out != nullptr, "coopmat_length: null output pointer");
    (void)dtype;   // the component count depends on the shape and use only
    int n = -1;
    if (use == LAVA_HIP_USE_ACCUMULATOR) {
        if (rows == 16 && cols == 16) n = length<Frag<float, 16, 16, Accumulator>>();
        else if (rows == 32 && cols == 32) n = length<Frag<float, 32, 32, Accumulator>>();
    } else if (use == LAVA_HIP_USE_MATRIX_A) {
        if (rows == 16 && cols == 16) n = length<Frag<lava::f16, 16, 16, MatrixA>>();
        else if (rows == 16 && cols == 32) n = length<Frag<lava::f16, 16, 32, MatrixA>>();
        else if (rows == 32 && cols == 16) n = length<Frag<lava::f16, 32, 16, MatrixA>>();
        else if (rows == 32 && cols == 32) n = length<Frag<lava::f16, 32, 32, MatrixA>>();
        else if (rows == 16 && cols == 64) n = length<Frag<int8_t, 16, 64, MatrixA>>();
    } else if (use == LAVA_HIP_USE_MATRIX_B) {
        if (rows == 16 && cols == 16) n = length<Frag<lava::f16, 16, 16, MatrixB>>();
        else if (rows == 32 && cols == 16) n = length<Frag<lava::f16, 32, 16, MatrixB>>();
        else if (rows == 16 && cols == 32) n = length<Frag<lava::f16, 16, 32, MatrixB>>();
        else if (rows == 32 && cols == 32) n = length<Frag<lava::f16, 32, 32, MatrixB>>();
        else if (rows == 64 && cols == 16) n = length<Frag<int8_t, 64, 16, MatrixB>>();
    }
    LAVA_REQUIRE(n > 0, LAVA_HIP_ERR_UNSUPPORTED, "coopmat_length: no %d x %d fragment of use %d", rows, cols, use);
    *length_out = n;
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_perelement_scale(const float* in, float* out, int tile, int by_row, const void* factors,
                                      int64_t base, int64_t ntiles, void* stream) {
    LAVA_ARG(tile == 16 || tile == 32, "coopmat_perelement_scale: tile = %d is not 16 or 32", tile);
    LAVA_ARG(ntiles >= 0 && ntiles <= 0x7fffffff, "coopmat_perelement_scale: ntiles out of range");
    if (ntiles == 0) return LAVA_HIP_OK;
    LAVA_ARG(in && out && factors, "coopmat_perelement_scale: null pointer");
    LAVA_ARG(base >= 0 && base + ntiles * tile <= 0xffffffffll, "coopmat_perelement_scale: base out of range");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    const dim3 g((unsigned)ntiles);
    hipStream_t s = as_stream(stream);
    const uint32_t b = (uint32_t)base;
    if (tile == 16 && by_row) hipLaunchKernelGGL((perelement_scale_kernel<16, true>), g, dim3(64), 0, s, in, out, factors, b);
    else if (tile == 16) hipLaunchKernelGGL((perelement_scale_kernel<16, false>), g, dim3(64), 0, s, in, out, factors, b);
    else if (by_row) hipLaunchKernelGGL((perelement_scale_kernel<32, true>), g, dim3(64), 0, s, in, out, factors, b);
    else hipLaunchKernelGGL((perelement_scale_kernel<32, false>), g, dim3(64), 0, s, in, out, factors, b);
    LAVA_LAUNCH_CHECK("perelement_scale_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_workgroup_shapes(int32_t* out, int max_rows, int* count) {
    LAVA_ARG(count != nullptr, "workgroup_shapes: null count pointer");
    const int n = (int)(sizeof(kWgShapes) / sizeof(kWgShapes[0]));
    *count = n;
    if (out == nullptr) return LAVA_HIP_OK;
    for (int i = 0; i < n && i < max_rows; ++i) {
        out[4 * i + 0] = kWgShapes[i].nt;
        out[4 * i + 1] = 16 * kWgShapes[i].wm;
        out[4 * i + 2] = 16 * kWgShapes[i].wn;
        out[4 * i + 3] = 16;
    }
    return LAVA_HIP_OK;
}

int lava_hip_coopmat_workgroup_gemm_f16(int invocations, const void* A, const void* B, float* C, int64_t M, int64_t N,
                                        int64_t K, int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout,
                                        void* stream) {
    int wm = 0, wn = 0;
    for (const WgShape& w : kWgShapes)
        if (w.nt == invocations) { wm = w.wm; wn = w.wn; }
    LAVA_REQUIRE(wm > 0, LAVA_HIP_ERR_UNSUPPORTED, "workgroup_gemm: no workgroup-scope matrix at %d invocations",
                 invocations);
    LAVA_ARG(layout <= 7u, "workgroup_gemm: layout %u has bits beyond A, B, C row-major", layout);
    LAVA_ARG(M > 0 && N > 0 && K > 0 && M % (16 * wm) == 0 && N % (16 * wn) == 0 && K % 16 == 0,
             "workgroup_gemm: (M, N, K) = (%lld, %lld, %lld) are not positive multiples of (%d, %d, 16) at %d invocations",
             (long long)M, (long long)N, (long long)K, 16 * wm, 16 * wn, invocations);
    LAVA_ARG(M <= 4096 && N <= 4096 && K <= 4096, "workgroup_gemm: one workgroup holds at most 4096 x 4096 x 4096");
    const bool arow = layout & 1u, brow = layout & 2u, crow = layout & 4u;
    LAVA_ARG(lda >= (arow ? K : M) && ldb >= (brow ? N : K) && ldc >= (crow ? N : M),
             "workgroup_gemm: leading dimension too small");
    LAVA_ARG(A && B && C, "workgroup_gemm: null pointer");
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipStream_t s = as_stream(stream);
    const dim3 blk((unsigned)(64 * wm * wn));
#define LAVA_WG(WM_, WN_)                                                                                        \
    hipLaunchKernelGGL((workgroup_gemm_kernel<WM_, WN_>), dim3(1), blk, 0, s, (const lava::f16*)A,              \
                       (const lava::f16*)B, C, (int)M, (int)N, (int)K, lda, ldb, ldc, layout)
    switch (invocations) {
    case 64: LAVA_WG(1, 1); break;
    case 128: LAVA_WG(2, 1); break;
    case 256: LAVA_WG(2, 2); break;
    case 512: LAVA_WG(4, 2); break;
    default: LAVA_WG(4, 4); break;
    }
#undef LAVA_WG
    LAVA_LAUNCH_CHECK("workgroup_gemm_kernel");
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
