// gemm_mid.hip -- the mid-size GEMM kernel's applicability and kernel-choice rule, and its plain
// (fp32 / int32 output) instances; the kernel is in gemm_mid_kernel.hpp, the fused-epilogue and
// unsigned-byte instances in gemm_mid_ex.hip.
#include "gemm_mid_kernel.hpp"

namespace lava {

template <typename T>
int mid_gemm_eligible(const void* A, const void* B, const void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc, size_t c_elem, bool ak, bool bk) {
    const int64_t sz = (int64_t)sizeof(T), ke = TN_KB / sz, chunk = 16 / sz;
    if (M <= 0 || N <= 0 || K <= 0) return TN_NO;
    if ((ak || bk) && K % chunk) return TN_NO;           // a K-contiguous chunk wholly in or out
    if ((!ak && M % chunk) || (!bk && N % chunk)) return TN_NO;
    const int64_t tiles_m = (M + TM_TILE - 1) / TM_TILE, tiles_n = (N + TM_TILE - 1) / TM_TILE;
    if (tiles_m * tiles_n > 0x7fffffff || (K + ke - 1) / ke > 0x7fffffff || K * sz > 0x7fffffff) return TN_NO;
    if ((lda * sz) % 16 || (ldb * sz) % 16 || !aligned(A, 16) || !aligned(B, 16)) return TN_NO;
    // buffer offsets are 32-bit: a 128-row K-contiguous slab, or the whole K x ld M/N-contiguous
    // operand, must span < 2 GiB
    const int64_t lim = (int64_t)1 << 31;
    if ((ak ? (int64_t)TM_TILE * lda * sz : K * lda * sz) >= lim) return TN_NO;
    if ((bk ? (int64_t)TM_TILE * ldb * sz : K * ldb * sz) >= lim) return TN_NO;
    if (M % TM_TILE == 0 && N % TM_TILE == 0 && K % ke == 0 && ldc % 4 == 0 && aligned(C, 4 * c_elem)) return TN_FULL;
    return TN_RAGGED;
}

// The automatic choice (measured, A row-major and B column-major, interleaved on one box; bf16
// TFLOP/s and int8 TOP/s, this kernel against the best of the others): 2048^3 667 / 410 and 1193 /
// 693, 2048 x 4096 x 4096 1149 / 901 and 1909 / 1567, 2048^2 x 8192 914 / 506, 1536^2 x 8192 543 /
// 338, 1024 x 4096 x 4096 773 / 471, 512 x 4096 x 4096 412 / 433 and 884 / 721 -- while the 256 x 256
// tile kernel keeps 3072^3 (948 against 766; 144 tiles) and 4096^3 (1406 against 1164), and the
// small-product kernel's K split 1024^2 x 8192 (383 against 245; 64 tiles of 128 x 128).  So: at
// least 128 tiles of 128 x 128, and fewer than 144 of 256 x 256.  With M/N-contiguous bf16 operands
// the same boundaries hold (A and B column-major: 2048^3 620 / 401, 2048 x 4096 x 4096 1104 / 812,
// 1536^2 x 8192 496 / 322, 3072^3 768 / 866, 1024^2 x 8192 221 / 374; A and B row-major or A
// column-major and B row-major within 6 % of these; int8 with A and B column-major 2048^3 1167 / 627,
// where the small kernel reads both operands through transposing LDS reads at 621 -- and at 1024^3, 64
// tiles, it leads, 242 against 225).  Past one full round of 256 x 256 tiles, a
// second round of at most 80 of them leaves this kernel ahead (bf16 TFLOP/s and int8 TOP/s, this
// kernel / the tile kernel: 3072 x 6144 x 4096, 288 tiles, 1037 / 933 and 1789 / 1620; 4096 x 5120 x
// 2048, 320 tiles, 986 / 906 and 1610 / 1453; 4608^2 x 4096, 324 tiles, 1073 / 1037 and 1855 / 1793;
// 4608^2 x 1024 780 / 730 and 1201 / 1045), a fuller one does not (6144 x 4096 x 4096, 384 tiles, 1187 /
// 1199 and 2002 / 2084; 5120^2 x 4096, 400, 1055 / 1237; 6144^2 x 4096, 576, 1151 / 1199).
bool mid_gemm_preferred(int64_t M, int64_t N) {
    const int64_t t128 = ((M + TM_TILE - 1) / TM_TILE) * ((N + TM_TILE - 1) / TM_TILE);
    const int64_t t256 = ((M + TN_TILE - 1) / TN_TILE) * ((N + TN_TILE - 1) / TN_TILE);
    return t128 >= 128 && (t256 < 144 || (t256 > 256 && t256 <= 336));
}

LAVA_MID_LAUNCH_INST(f16, float, false, false)
LAVA_MID_LAUNCH_INST(bf16, float, false, false)
LAVA_MID_LAUNCH_INST(int8_t, int32_t, false, false)
template int mid_gemm_eligible<f16>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t, int64_t,
                                    int64_t, size_t, bool, bool);
template int mid_gemm_eligible<bf16>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t,
                                     int64_t, int64_t, size_t, bool, bool);
template int mid_gemm_eligible<int8_t>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t,
                                       int64_t, int64_t, size_t, bool, bool);

}  // namespace lava
