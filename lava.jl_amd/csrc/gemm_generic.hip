// gemm_generic.hip -- GEMM kernels for every layout and any shape.
//
//  * gemm_staged_kernel: 64x64 output tile per workgroup of 4 wavefronts, one
//    K-slice of 64 bytes staged through LDS with bounds-predicated loads, so it
//    covers row- and column-major A and B and extents that are not tile
//    multiples (the clamp-to-zero of a TENSOR_CLAMP_CONSTANT load,
//    src/vocabulary/tensor.jl:46-51).  It is the fallback behind the fast TN
//    kernel and the path for small problems.
//  * coopmat_tiles_kernel: the 16x16x16 subgroup-tile GEMM written in the
//    vocabulary exactly as docs/src/device.md:81-88 writes it -- one wavefront per
//    tile of C, fragments loaded straight from global memory.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gemm_common.hpp"
#include "gemm_kernels.hpp"
#include "lava_hip_internal.hpp"

namespace lava {

template <typename T, bool AROW, bool BROW, typename OutT, bool EPI>
__global__ void __launch_bounds__(256) gemm_staged_kernel(const T* __restrict__ A, const T* __restrict__ B,
                                                          OutT* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                          int64_t lda, int64_t ldb, int64_t ldc, Epilogue epi) {
    using Acc = typename Mfma16<T>::acc_elem;
    using AccV = typename Mfma16<T>::acc_t;
    constexpr int KE = Mfma16<T>::k;        // elements per K-slice (64 bytes)
    constexpr int ROWB = 80;                // 64 data bytes + 16 bytes of padding per LDS row
    constexpr int PER = 64 * KE / 256;      // elements per thread per operand
    __shared__ __attribute__((aligned(16))) uint8_t As[64 * ROWB];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[64 * ROWB];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
    const int wm = w >> 1, wn = w & 1;
    AccV acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = AccV{0, 0, 0, 0};

    for (int64_t k0 = 0; k0 < K; k0 += KE) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = tid + 256 * i;
            int r, kk;
            if (AROW) { r = e / KE; kk = e % KE; }
            else { kk = e / 64; r = e % 64; }
            const int64_t gm = m0 + r, gk = k0 + kk;
            T v = (T)0;
            if (gm < M && gk < K) v = AROW ? A[gm * lda + gk] : A[gk * lda + gm];
            *reinterpret_cast<T*>(As + r * ROWB + kk * (int)sizeof(T)) = v;
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = tid + 256 * i;
            int n, kk;
            if (BROW) { kk = e / 64; n = e % 64; }
            else { n = e / KE; kk = e % KE; }
            const int64_t gn = n0 + n, gk = k0 + kk;
            T v = (T)0;
            if (gn < N && gk < K) v = BROW ? B[gk * ldb + gn] : B[gn * ldb + gk];
            *reinterpret_cast<T*>(Bs + n * ROWB + kk * (int)sizeof(T)) = v;
        }
        __syncthreads();
        uint4 af[2], bf[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            af[t] = *reinterpret_cast<const uint4*>(As + (wm * 32 + t * 16 + (lane & 15)) * ROWB + (lane >> 4) * 16);
            bf[t] = *reinterpret_cast<const uint4*>(Bs + (wn * 32 + t * 16 + (lane & 15)) * ROWB + (lane >> 4) * 16);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = Mfma16<T>::run(af[i], bf[j], acc[i][j]);
        __syncthreads();
    }
    // lane holds column lane % 16 and rows 4 * (lane / 16) + q of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t gn = n0 + wn * 32 + j * 16 + (lane & 15);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t gm = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + q;
                if (gm < M && gn < N) {
                    if constexpr (!EPI && std::is_same<OutT, Acc>::value)
                        C[gm * ldc + gn] = (Acc)acc[i][j][q];
                    else
                        C[gm * ldc + gn] =
                            narrow<OutT>(EPI ? epi_apply(epi, gm, gn, (float)acc[i][j][q]) : (float)acc[i][j][q]);
                }
            }
        }
}

__global__ void __launch_bounds__(256) coopmat_tiles_kernel(const f16* __restrict__ A, const f16* __restrict__ B,
                                                            float* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                            int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout) {
    const bool arow = (layout & 1u) != 0, brow = (layout & 2u) != 0, crow = (layout & 4u) != 0;
    const int64_t tiles_n = N / 16;
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave >= (M / 16) * tiles_n) return;  // whole wavefront leaves together
    const int64_t tm = wave / tiles_n, tn = wave % tiles_n;
    auto c = zero<Frag<float, 16, 16, Accumulator>>();
    for (int64_t k = 0; k < K; k += 16) {
        auto a = load<Frag<f16, 16, 16, MatrixA>>(A + (arow ? tm * 16 * lda + k : k * lda + tm * 16), lda, arow);
        auto b = load<Frag<f16, 16, 16, MatrixB>>(B + (brow ? k * ldb + tn * 16 : tn * 16 * ldb + k), ldb, brow);
        c = mma(a, b, c);
    }
    store(C + (crow ? tm * 16 * ldc + tn * 16 : tn * 16 * ldc + tm * 16), ldc, crow, c);
}

template <typename T, typename OutT, bool EPI>
int launch_gemm_staged(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                       int64_t ldc, bool arow, bool brow, hipStream_t s, const Epilogue& epi) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (arow && brow)
        hipLaunchKernelGGL((gemm_staged_kernel<T, true, true, OutT, EPI>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi);
    else if (arow)
        hipLaunchKernelGGL((gemm_staged_kernel<T, true, false, OutT, EPI>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi);
    else if (brow)
        hipLaunchKernelGGL((gemm_staged_kernel<T, false, true, OutT, EPI>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi);
    else
        hipLaunchKernelGGL((gemm_staged_kernel<T, false, false, OutT, EPI>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi);
    LAVA_LAUNCH_CHECK("gemm_staged_kernel");
    return LAVA_HIP_OK;
}

#define LAVA_STAGED_INST(T, O, E)                                                                              \
    template int launch_gemm_staged<T, O, E>(const T*, const T*, O*, int64_t, int64_t, int64_t, int64_t, int64_t, \
                                             int64_t, bool, bool, hipStream_t, const Epilogue&);
LAVA_STAGED_INST(f16, float, false)
LAVA_STAGED_INST(bf16, float, false)
LAVA_STAGED_INST(int8_t, int32_t, false)
LAVA_STAGED_INST(f16, float, true)
LAVA_STAGED_INST(f16, f16, true)
LAVA_STAGED_INST(f16, bf16, true)
LAVA_STAGED_INST(bf16, float, true)
LAVA_STAGED_INST(bf16, f16, true)
LAVA_STAGED_INST(bf16, bf16, true)
#undef LAVA_STAGED_INST

int launch_coopmat_tiles(const f16* A, const f16* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, uint32_t layout, hipStream_t s) {
    const int64_t waves = (M / 16) * (N / 16);
    const int64_t blocks = (waves + 3) / 4;
    if (blocks == 0) return LAVA_HIP_OK;
    hipLaunchKernelGGL(coopmat_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, ldc,
                       layout);
    LAVA_LAUNCH_CHECK("coopmat_tiles_kernel");
    return LAVA_HIP_OK;
}

}  // namespace lava
