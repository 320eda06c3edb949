// gemm_tn.hip -- the compute-bound GEMM: A row-major, B column-major, C row-major.
//
// This is the staged cooperative-matrix GEMM (src/device/coopmat_intrinsics.jl:
// 104-148 stages A and B through workgroup memory and reads A RowMajor and B
// ColumnMajor from the same block; test/glsl/coopmat2_gemm_regs.comp:46-84 is the
// same loop at workgroup scope) laid out for CDNA4:
//
//  * one 256 x 256 tile of C per workgroup of 4 wavefronts (one per SIMD), each
//    wavefront owning a 128 x 128 sub-tile = 8 x 8 MFMA 16x16 accumulators
//    (256 fp32 registers per lane);
//  * K advances 128 bytes at a time (64 bf16/fp16 or 128 int8): A and B slices of
//    256 rows x 128 bytes each, double-buffered in LDS (2 x 64 KB);
//  * global -> LDS with global_load_lds_dwordx4: each lane moves 16 bytes straight
//    into LDS, no register staging.  One wavefront instruction fills 1 KB = 8 LDS
//    rows; lane l writes row l / 8, 16-byte slot l % 8.  The slot a logical 16-byte
//    chunk c of row r lands in is c ^ swz(r), swz(r) = (r & 7) ^ ((r >> 3) & 1),
//    chosen by which global chunk each lane fetches, so the fragment reads
//    (16 consecutive rows, one chunk column) spread over all banks;
//  * fragments are 16 bytes per lane (ds_read_b128), one MFMA 16x16x32 (16-bit)
//    or 16x16x64 (int8) each;
//  * the MFMA's A operand is the B slice and its B operand the A slice, so each
//    lane's accumulator holds 4 consecutive columns of one row of C: the epilogue
//    is one 16-byte store per lane per accumulator;
//  * workgroups are renumbered XCD by XCD (xcd_tile) so that the tiles one XCD
//    runs together share rows of A and columns of B in its L2.
#include <hip/hip_runtime.h>

#include "gemm_common.hpp"
#include "gemm_kernels.hpp"
#include "lava_hip_internal.hpp"

namespace lava {

constexpr int TN_TILE = 256;    // rows of A / columns of B per workgroup
constexpr int TN_KB = 128;      // bytes of K per stage
constexpr int TN_SLICE = TN_TILE * TN_KB;  // 32 KB

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(const void* gsrc, lds_void* ldst) {
    __builtin_amdgcn_global_load_lds(gsrc, ldst, 16, 0, 0);
}

template <typename T>
__global__ void __launch_bounds__(256, 1)
    gemm_tn_kernel(const T* __restrict__ A, const T* __restrict__ B, typename Mfma16<T>::acc_elem* __restrict__ C,
                   int tiles_m, int tiles_n, int ktiles, int64_t lda_b, int64_t ldb_b, int64_t ldc) {
    using AccV = typename Mfma16<T>::acc_t;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * 2 * TN_SLICE];  // [stage][A,B][row][128 B]

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int tm, tn;
    xcd_tile(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);

    // ---- global -> LDS: wave w fills rows [64w, 64w + 64) of each slice, 8 rows per instruction.
    // Instruction i covers rows 64w + 8i + lane / 8; lane's slot is lane % 8; the
    // logical chunk fetched is slot ^ swz(row) = (lane % 8) ^ (lane / 8) ^ (i & 1).
    const int lr = lane >> 3;
    const int c_even = (lane & 7) ^ lr;
    const int c_odd = c_even ^ 1;
    const char* a_src = reinterpret_cast<const char*>(A) + ((int64_t)tm * TN_TILE + 64 * w + lr) * lda_b;
    const char* b_src = reinterpret_cast<const char*>(B) + ((int64_t)tn * TN_TILE + 64 * w + lr) * ldb_b;
    const int64_t a_step = 8 * lda_b, b_step = 8 * ldb_b;

    auto issue = [&](int stage, int kt) {
        uint8_t* a_dst = smem + stage * 2 * TN_SLICE + w * 64 * TN_KB;
        uint8_t* b_dst = a_dst + TN_SLICE;
        const int64_t kofs = (int64_t)kt * TN_KB;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = (i & 1) ? c_odd : c_even;
            dma16(a_src + i * a_step + kofs + c * 16, (lds_void*)(a_dst + i * 1024));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = (i & 1) ? c_odd : c_even;
            dma16(b_src + i * b_step + kofs + c * 16, (lds_void*)(b_dst + i * 1024));
        }
    };

    // ---- fragment reads: row = base + 16 t + lane % 16; chunk = 4 s + lane / 16.
    // swz(row) only depends on lane % 16, so every read of a lane uses one slot per s.
    const int wm = w >> 1, wn = w & 1;
    const int swz = (lane & 7) ^ ((lane >> 3) & 1);
    const int rd_row = lane & 15;
    const int slot0 = (0 + (lane >> 4)) ^ swz;
    const int slot1 = (4 + (lane >> 4)) ^ swz;
    const int a_rd = (wm * 128 + rd_row) * TN_KB;
    const int b_rd = TN_SLICE + (wn * 128 + rd_row) * TN_KB;

    AccV acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = AccV{0, 0, 0, 0};

    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    for (int kt = 0; kt < ktiles; ++kt) {
        const int stage = kt & 1;
        if (kt + 1 < ktiles) issue(stage ^ 1, kt + 1);
        const uint8_t* base = smem + stage * 2 * TN_SLICE;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int slot = s ? slot1 : slot0;
            uint4 af[8], bf[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                af[t] = *reinterpret_cast<const uint4*>(base + a_rd + t * 16 * TN_KB + slot * 16);
                bf[t] = *reinterpret_cast<const uint4*>(base + b_rd + t * 16 * TN_KB + slot * 16);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = Mfma16<T>::run(bf[j], af[i], acc[i][j]);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }

    // ---- epilogue: acc[i][j] lane holds C[m][n .. n + 3] with
    // m = tile row + 128 wm + 16 i + lane % 16, n = tile col + 128 wn + 16 j + 4 (lane / 16).
    typedef typename Mfma16<T>::acc_elem Acc;
    Acc* crow = C + ((int64_t)tm * TN_TILE + wm * 128 + (lane & 15)) * ldc + (int64_t)tn * TN_TILE + wn * 128 +
                4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) *reinterpret_cast<AccV*>(crow + (int64_t)i * 16 * ldc + j * 16) = acc[i][j];
}

template <typename T>
bool tn_gemm_eligible(const void* A, const void* B, const void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc) {
    const int64_t ke = TN_KB / (int64_t)sizeof(T);
    if (M <= 0 || N <= 0 || K <= 0) return false;
    if (M % TN_TILE || N % TN_TILE || K % ke) return false;
    if ((M / TN_TILE) * (N / TN_TILE) > 0x7fffffff || K / ke > 0x7fffffff) return false;
    if ((lda * (int64_t)sizeof(T)) % 16 || (ldb * (int64_t)sizeof(T)) % 16 || ldc % 4) return false;
    if (!aligned(A, 16) || !aligned(B, 16) || !aligned(C, 16)) return false;
    return true;
}

template <typename T>
int launch_gemm_tn(const T* A, const T* B, typename Mfma16<T>::acc_elem* C, int64_t M, int64_t N, int64_t K,
                   int64_t lda, int64_t ldb, int64_t ldc, hipStream_t s) {
    const int tiles_m = (int)(M / TN_TILE), tiles_n = (int)(N / TN_TILE);
    const int ktiles = (int)(K / (TN_KB / (int64_t)sizeof(T)));
    hipLaunchKernelGGL(gemm_tn_kernel<T>, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, s, A, B, C, tiles_m,
                       tiles_n, ktiles, lda * (int64_t)sizeof(T), ldb * (int64_t)sizeof(T), ldc);
    LAVA_LAUNCH_CHECK("gemm_tn_kernel");
    return LAVA_HIP_OK;
}

template bool tn_gemm_eligible<f16>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t, int64_t,
                                    int64_t);
template bool tn_gemm_eligible<bf16>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t,
                                     int64_t, int64_t);
template bool tn_gemm_eligible<int8_t>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t,
                                       int64_t, int64_t);
template int launch_gemm_tn<f16>(const f16*, const f16*, float*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                 hipStream_t);
template int launch_gemm_tn<bf16>(const bf16*, const bf16*, float*, int64_t, int64_t, int64_t, int64_t, int64_t,
                                  int64_t, hipStream_t);
template int launch_gemm_tn<int8_t>(const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t, int64_t,
                                    int64_t, int64_t, hipStream_t);

}  // namespace lava
