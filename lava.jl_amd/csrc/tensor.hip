// tensor.hip -- tensor addressing: the vocabulary entry points and the coopmat2 GEMM.
//
//  * lava_hip_tensor_load_tile / lava_hip_tensor_store_tile: one fragment through a
//    TensorLayout (and the transposing TensorView), so that the clamp modes, the
//    clamp value, slices and views can be checked element by element;
//  * lava_hip_tensor_muladd_16x16x16: D = A * B with both operands loaded through
//    layouts -- e.g. the V operand of attention padded with a clamp value of one,
//    whose padding columns of P * V then hold the row sums of P
//    (src/device/tensor_intrinsics.jl:139-155);
//  * lava_hip_gemm_cm2_f16: the coopmat2 GEMM of test/glsl/coopmat2_gemm_regs.comp:
//    37-84 (fp16 A, B row-major, zero-clamped so that any M, N, K works unpadded, fp16
//    C stored plainly or through the transposing view).  By default it runs on the
//    256 x 256 tile kernel, whose buffer-resource loads are this hardware's clamping
//    tensor layout (a lane past the extent reads zero); LAVA_HIP_CM2_VOCABULARY runs
//    the shader's own form written in the tensor vocabulary below: workgroups of 256
//    invocations own a 128 x 128 block of C, K advances 64 at a time, A and B are
//    tensor_load-ed straight from memory through layouts sliced per block, the fp32
//    sum is converted to fp16 and tensor_store-d through a clamping layout or the
//    (1, 0) view.  The shader's one workgroup-scope 128 x 128 matrix is held as 4
//    wavefronts x (2 x 2) 32 x 32 MFMA accumulators.
#include <hip/hip_runtime.h>

#include "lava_hip_internal.hpp"
#include "lava_tensor.hpp"

namespace lava {
namespace {

// ---- one fragment through a layout ------------------------------------------------
template <typename T, int R, int C, Use U, bool TRANS>
__global__ void __launch_bounds__(64) tensor_load_tile_kernel(const T* src, TensorLayout<4> l, const T* object,
                                                              T* out) {
    using F = Frag<T, R, C, U>;
    F m = load<F>(object, C, true);
    m = tensor_load<TRANS>(m, src, l);
    store(out, C, true, m);
}

template <typename T, int R, int C, Use U, bool TRANS>
__global__ void __launch_bounds__(64) tensor_store_tile_kernel(const T* in, T* dst, TensorLayout<4> l) {
    using F = Frag<T, R, C, U>;
    const F m = load<F>(in, C, true);
    tensor_store<TRANS>(m, dst, l);
}

template <bool TB>
__global__ void __launch_bounds__(64) tensor_muladd_kernel(const f16* A, TensorLayout<4> la, const f16* B,
                                                           TensorLayout<4> lb, float* D) {
    const auto a = tensor_load(zero<Frag<f16, 16, 16, MatrixA>>(), A, la);
    const auto b = tensor_load<TB>(zero<Frag<f16, 16, 16, MatrixB>>(), B, lb);
    const auto d = mma(a, b, zero<Frag<float, 16, 16, Accumulator>>());
    store(D, 16, true, d);
}

// ---- the coopmat2 GEMM ----------------------------------------------------------------
constexpr int CM2_BM = 128, CM2_BN = 128, CM2_BK = 64;

template <bool TRANS_C>
__global__ void __launch_bounds__(256) gemm_cm2_kernel(const f16* __restrict__ A, const f16* __restrict__ B,
                                                       f16* __restrict__ C, int M, int N, int K, int lda, int ldb,
                                                       int ldc) {
    const int ir = blockIdx.x, ic = blockIdx.y;
    const int w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
    const int32_t da[2] = {M, K}, sa[2] = {lda, 1}, db[2] = {K, N}, sb[2] = {ldb, 1};
    const TensorLayout<2> tlA = tensor_setstride(tensor_layout<2>(ClampConstant, da), sa);
    const TensorLayout<2> tlB = tensor_setstride(tensor_layout<2>(ClampConstant, db), sb);
    const int m0 = ir * CM2_BM + 64 * wm, n0 = ic * CM2_BN + 64 * wn;

    Frag<float, 32, 32, Accumulator> sum[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) sum[i][j] = zero<Frag<float, 32, 32, Accumulator>>();

    for (int block_k = 0; block_k < K; block_k += CM2_BK) {
#pragma unroll
        for (int kk = 0; kk < CM2_BK; kk += 16) {
            Frag<f16, 32, 16, MatrixA> a[2];
            Frag<f16, 16, 32, MatrixB> b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int32_t o[2] = {m0 + 32 * i, block_k + kk}, z[2] = {32, 16};
                a[i] = tensor_load(zero<Frag<f16, 32, 16, MatrixA>>(), A, tensor_slice(tlA, o, z));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int32_t o[2] = {block_k + kk, n0 + 32 * j}, z[2] = {16, 32};
                b[j] = tensor_load(zero<Frag<f16, 16, 32, MatrixB>>(), B, tensor_slice(tlB, o, z));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) sum[i][j] = mma(a[i], b[j], sum[i][j]);
        }
    }

    // C (M x N) through a clamping layout, or C^T (N x M) through the (1, 0) view
    const int32_t dc[2] = {TRANS_C ? N : M, TRANS_C ? M : N}, sc[2] = {ldc, 1};
    const TensorLayout<2> tlC = tensor_setstride(tensor_layout<2>(ClampConstant, dc), sc);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const Frag<f16, 32, 32, Accumulator> out16 = convert<f16>(sum[i][j]);
            const int r0 = m0 + 32 * i, c0 = n0 + 32 * j;
            const int32_t o[2] = {TRANS_C ? c0 : r0, TRANS_C ? r0 : c0}, z[2] = {32, 32};
            tensor_store<TRANS_C>(out16, C, tensor_slice(tlC, o, z));
        }
}

// ---- host helpers ---------------------------------------------------------------------
// A rank-r layout as rank 4: outer dimensions of extent 1, slice size 1, offset 0.
int to_layout4(const lava_hip_tensor_layout* in, TensorLayout<4>* out, const char* name) {
    LAVA_ARG(in != nullptr, "%s: null layout", name);
    LAVA_ARG(in->rank >= 2 && in->rank <= 4, "%s: layout rank %d is not 2, 3 or 4", name, in->rank);
    LAVA_ARG(in->clamp <= LAVA_HIP_CLAMP_TO_EDGE, "%s: unknown clamp mode %u", name, in->clamp);
    const int pad = 4 - in->rank;
    for (int d = 0; d < 4; ++d) {
        if (d < pad) {
            out->dim[d] = 1;
            out->stride[d] = 0;
            out->off[d] = 0;
            out->size[d] = 1;
            continue;
        }
        const int s = d - pad;
        LAVA_ARG(in->dim[s] >= 0 && in->size[s] >= 0, "%s: negative extent or slice size in dimension %d", name, s);
        out->dim[d] = in->dim[s];
        out->stride[d] = in->stride[s];
        out->off[d] = in->off[s];
        out->size[d] = in->size[s];
        if (d < 2) LAVA_ARG(in->size[s] == 1, "%s: the matrix maps onto the last two dimensions; slice size %d in "
                                              "outer dimension %d must be 1", name, in->size[s], s);
    }
    out->clamp = in->clamp;
    out->clampbits = in->clampbits;
    return LAVA_HIP_OK;
}

template <typename T, int R, int C, Use U>
void launch_tile(bool store_op, bool trans, const void* src_or_in, void* dst, const TensorLayout<4>& l,
                 const void* object, void* out, hipStream_t s) {
    if (!store_op) {
        if (trans)
            hipLaunchKernelGGL((tensor_load_tile_kernel<T, R, C, U, true>), dim3(1), dim3(64), 0, s,
                               (const T*)src_or_in, l, (const T*)object, (T*)out);
        else
            hipLaunchKernelGGL((tensor_load_tile_kernel<T, R, C, U, false>), dim3(1), dim3(64), 0, s,
                               (const T*)src_or_in, l, (const T*)object, (T*)out);
    } else {
        if (trans)
            hipLaunchKernelGGL((tensor_store_tile_kernel<T, R, C, U, true>), dim3(1), dim3(64), 0, s,
                               (const T*)src_or_in, (T*)dst, l);
        else
            hipLaunchKernelGGL((tensor_store_tile_kernel<T, R, C, U, false>), dim3(1), dim3(64), 0, s,
                               (const T*)src_or_in, (T*)dst, l);
    }
}

template <typename T>
void launch_tile_shape(int shape, bool store_op, bool trans, const void* a, void* dst, const TensorLayout<4>& l,
                       const void* object, void* out, hipStream_t s) {
    switch (shape) {
    case LAVA_HIP_TILE_A_16x16: launch_tile<T, 16, 16, MatrixA>(store_op, trans, a, dst, l, object, out, s); break;
    case LAVA_HIP_TILE_B_16x16: launch_tile<T, 16, 16, MatrixB>(store_op, trans, a, dst, l, object, out, s); break;
    case LAVA_HIP_TILE_ACC_16x16:
        launch_tile<T, 16, 16, Accumulator>(store_op, trans, a, dst, l, object, out, s);
        break;
    case LAVA_HIP_TILE_ACC_32x32:
        launch_tile<T, 32, 32, Accumulator>(store_op, trans, a, dst, l, object, out, s);
        break;
    case LAVA_HIP_TILE_A_32x16: launch_tile<T, 32, 16, MatrixA>(store_op, trans, a, dst, l, object, out, s); break;
    default: launch_tile<T, 16, 32, MatrixB>(store_op, trans, a, dst, l, object, out, s); break;
    }
}

int tile_entry(const char* name, bool store_op, int dtype, int shape, const void* a, void* dst,
               const lava_hip_tensor_layout* layout, int transpose, const void* object, void* out, void* stream) {
    LAVA_REQUIRE(dtype == LAVA_HIP_F16 || dtype == LAVA_HIP_F32, LAVA_HIP_ERR_UNSUPPORTED,
                 "%s: dtype %d is not F16 or F32", name, dtype);
    LAVA_ARG(shape >= LAVA_HIP_TILE_A_16x16 && shape <= LAVA_HIP_TILE_B_16x32, "%s: unknown tile shape %d", name,
             shape);
    LAVA_ARG(a != nullptr && (store_op ? dst != nullptr : (object != nullptr && out != nullptr)), "%s: null pointer",
             name);
    TensorLayout<4> l;
    int rc = to_layout4(layout, &l, name);
    if (rc != LAVA_HIP_OK) return rc;
    rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipStream_t s = as_stream(stream);
    if (dtype == LAVA_HIP_F16)
        launch_tile_shape<f16>(shape, store_op, transpose != 0, a, dst, l, object, out, s);
    else
        launch_tile_shape<float>(shape, store_op, transpose != 0, a, dst, l, object, out, s);
    LAVA_LAUNCH_CHECK(store_op ? "tensor_store_tile_kernel" : "tensor_load_tile_kernel");
    return LAVA_HIP_OK;
}

}  // namespace
}  // namespace lava

using namespace lava;

extern "C" {

int lava_hip_tensor_load_tile(int dtype, int shape, const void* src, const lava_hip_tensor_layout* layout,
                              int transpose, const void* object, void* out, void* stream) {
    return tile_entry("tensor_load_tile", false, dtype, shape, src, nullptr, layout, transpose, object, out, stream);
}

int lava_hip_tensor_store_tile(int dtype, int shape, const void* in, void* dst, const lava_hip_tensor_layout* layout,
                               int transpose, void* stream) {
    return tile_entry("tensor_store_tile", true, dtype, shape, in, dst, layout, transpose, nullptr, nullptr, stream);
}

int lava_hip_tensor_muladd_16x16x16(const void* A, const lava_hip_tensor_layout* layout_a, const void* B,
                                    const lava_hip_tensor_layout* layout_b, int transpose_b, float* D, void* stream) {
    LAVA_ARG(A && B && D, "tensor_muladd_16x16x16: null pointer");
    TensorLayout<4> la, lb;
    int rc = to_layout4(layout_a, &la, "tensor_muladd_16x16x16");
    if (rc != LAVA_HIP_OK) return rc;
    rc = to_layout4(layout_b, &lb, "tensor_muladd_16x16x16");
    if (rc != LAVA_HIP_OK) return rc;
    rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipStream_t s = as_stream(stream);
    if (transpose_b)
        hipLaunchKernelGGL(tensor_muladd_kernel<true>, dim3(1), dim3(64), 0, s, (const f16*)A, la, (const f16*)B, lb,
                           D);
    else
        hipLaunchKernelGGL(tensor_muladd_kernel<false>, dim3(1), dim3(64), 0, s, (const f16*)A, la, (const f16*)B, lb,
                           D);
    LAVA_LAUNCH_CHECK("tensor_muladd_kernel");
    return LAVA_HIP_OK;
}

int lava_hip_gemm_cm2_f16(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t flags, void* stream) {
    LAVA_ARG((flags & ~(LAVA_HIP_CM2_TRANSPOSE_C | LAVA_HIP_CM2_VOCABULARY)) == 0, "gemm_cm2_f16: unknown flags 0x%x",
             flags);
    const bool transpose_c = flags & LAVA_HIP_CM2_TRANSPOSE_C;
    LAVA_ARG(M >= 0 && N >= 0 && K >= 0, "gemm_cm2_f16: negative extent");
    if (M == 0 || N == 0) return LAVA_HIP_OK;
    LAVA_ARG(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff && lda <= 0x7fffffff && ldb <= 0x7fffffff &&
                 ldc <= 0x7fffffff,
             "gemm_cm2_f16: extents and leading dimensions are 32-bit in a tensor layout");
    LAVA_ARG(C != nullptr && (K == 0 || (A != nullptr && B != nullptr)), "gemm_cm2_f16: null pointer");
    LAVA_ARG(lda >= (K > 0 ? K : 1) && ldb >= N && ldc >= (transpose_c ? M : N),
             "gemm_cm2_f16: leading dimension too small (lda >= K, ldb >= N, ldc >= %s)", transpose_c ? "M" : "N");
    LAVA_ARG(aligned(A, 2) && aligned(B, 2) && aligned(C, 2), "gemm_cm2_f16: operands not 2-byte aligned");
    const int64_t gx = (M + CM2_BM - 1) / CM2_BM, gy = (N + CM2_BN - 1) / CM2_BN;
    LAVA_ARG(gx <= 0x7fffffff && gy <= 65535, "gemm_cm2_f16: N = %lld needs more than 65535 workgroup columns",
             (long long)N);
    if (!(flags & LAVA_HIP_CM2_VOCABULARY))   // the 256 x 256 tile kernel: zero-clamped buffer loads
        return lava_hip_gemm_ex(LAVA_HIP_F16, LAVA_HIP_F16, A, B, C, M, N, K, lda, ldb, ldc,
                                LAVA_HIP_A_ROWMAJOR | LAVA_HIP_B_ROWMAJOR | (transpose_c ? 0u : LAVA_HIP_C_ROWMAJOR),
                                nullptr, nullptr, 0, LAVA_HIP_ACT_NONE, stream);
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    hipStream_t s = as_stream(stream);
    if (transpose_c)
        hipLaunchKernelGGL(gemm_cm2_kernel<true>, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, s, (const f16*)A,
                           (const f16*)B, (f16*)C, (int)M, (int)N, (int)K, (int)lda, (int)ldb, (int)ldc);
    else
        hipLaunchKernelGGL(gemm_cm2_kernel<false>, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, s, (const f16*)A,
                           (const f16*)B, (f16*)C, (int)M, (int)N, (int)K, (int)lda, (int)ldb, (int)ldc);
    LAVA_LAUNCH_CHECK("gemm_cm2_kernel");
    return LAVA_HIP_OK;
}

}  // extern "C"
