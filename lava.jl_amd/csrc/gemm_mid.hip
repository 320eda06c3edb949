// gemm_mid.hip -- the mid-size GEMM kernel (gemm_mid_kernel): 128 x 128 tiles of C, for products
// whose 256 x 256 tiles would leave most of the 256 CUs idle (2048^3: 64 of them, against 256
// tiles of 128 x 128) and that the 64 x 64 small-product kernel runs well below the matrix
// cores' rate.  f16, bf16 or int8, each operand K-contiguous (A row-major, B column-major) or
// M/N-contiguous; plain fp32 / int32 output.  The staging is the tile kernel's at 128 rows
// (gemm_tn_kernel.hpp: TnSide<T, true, 128>, LDS-DMA of 128 bytes of K per m or n row, chunk ^ row %
// 8; TnSide<T, false, 128>, 128 bytes of K as rows of 128 m or n, read back transposed) on a quarter
// of its LDS, so that two workgroups share a CU and their wavefronts interleave on each SIMD:
//  * 4 wavefronts, each a 64 x 64 sub-tile = 4 x 4 16x16 accumulators (64 registers per lane);
//  * K advances 128 bytes per k-tile: A and B slices of 16 KB each, double-buffered (64 KB);
//  * per k-tile, as in the tile kernel: 16 MFMAs of k-step 0 with k-step 1's 8 fragment reads,
//    the barrier (this wavefront's DMAs of the next tile landed), 16 MFMAs of k-step 1 with the
//    next tile's k-step 0 reads and the 8 DMAs of the tile after next;
//  * the epilogue stages 32 rows x 64 columns per wavefront at a time through LDS and stores whole
//    256-byte row runs (4 rows per instruction), nontemporal.
#include "gemm_tn_kernel.hpp"

namespace lava {

constexpr int TM_TILE = 128;
constexpr int TM_SLICE = TM_TILE * TN_KB;   // 16 KB

template <typename T, bool RAGGED, bool AK, bool BK>
__global__ void __launch_bounds__(256, 2)
    gemm_mid_kernel(const T* __restrict__ A, const T* __restrict__ B, typename Mfma16<T>::acc_elem* __restrict__ C,
                    int tiles_m, int tiles_n, int ktiles, int64_t lda_b, int64_t ldb_b, int64_t ldc, TnBounds bnd) {
    using AccV = typename Mfma16<T>::acc_t;
    typedef typename Mfma16<T>::acc_elem Acc;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * 2 * TM_SLICE];   // [stage][A, B][16 KB]

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int tm, tn;
    xcd_tile(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
    const int wm = w >> 1, wn = w & 1;

    // rows (m, n) of this tile inside the matrix: all 128 unless RAGGED and the tile is the last
    int a_rows = TM_TILE, b_rows = TM_TILE;
    if constexpr (RAGGED) {
        a_rows = (int)(bnd.m - (int64_t)tm * TM_TILE < TM_TILE ? bnd.m - (int64_t)tm * TM_TILE : TM_TILE);
        b_rows = (int)(bnd.n - (int64_t)tn * TM_TILE < TM_TILE ? bnd.n - (int64_t)tn * TM_TILE : TM_TILE);
    }
    const int kelems = bnd.kb / (int)sizeof(T);
    TnSide<T, AK, TM_TILE> sa;
    TnSide<T, BK, TM_TILE> sb;
    sa.init(A, lda_b, tm, a_rows, bnd.m, kelems, w, wm, lane);
    sb.init(B, ldb_b, tn, b_rows, bnd.n, kelems, w, wn, lane);
    // wave w fills bytes [4 KB w, 4 KB (w + 1)) of each slice (32 m / n rows, or 16 k rows), instruction i 1 KB of it
    const uint32_t lds0 = lds_addr(smem) + w * (TM_TILE / 4) * TN_KB;

    // DMA load q (0..7) of a k-tile into `stage`: q < 4 are A, q >= 4 B.
    auto dma = [&](int q, int stage, uint32_t kofs) {
        const int i = q & 3;
        const uint32_t dst = lds0 + stage * 2 * TM_SLICE + (q >> 2) * TM_SLICE + i * 1024;
        if (q < 4) {
            uint32_t off = sa.voff(i);
            if constexpr (RAGGED) off = sa.valid(i, kofs, bnd.kb) ? off : OOB_OFS;
            dma16(sa.rs, off, sa.soff(i, kofs), dst);
        } else {
            uint32_t off = sb.voff(i);
            if constexpr (RAGGED) off = sb.valid(i, kofs, bnd.kb) ? off : OOB_OFS;
            dma16(sb.rs, off, sb.soff(i, kofs), dst);
        }
    };

    AccV acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0;

    // fragments of one k-step: a[i] rows 16 i of the wavefront's 64 m, b[j] rows 16 j of its 64 n
    struct F8 {
        uint4 a[4], b[4];
    };
    // fragment t (0..7) of k-step u, in the order the MFMAs (i-major) first use them: a[0], b[0..3], a[1..3]
    auto rd8 = [&](F8& f, const uint8_t* stage, int u, int t) {
        const bool isa = t == 0 || t > 4;
        const int blk = t == 0 ? 0 : (t <= 4 ? t - 1 : t - 4);
        if (isa) f.a[blk] = sa.read16(stage, u, blk);
        else f.b[blk] = sb.read16(stage + TM_SLICE, u, blk);
    };
    // MFMA A operand = B fragment, B operand = A fragment: acc[i][j] register r of lane l is
    // C[m][n], m = 64 wm + 16 i + l % 16, n = 64 wn + 16 j + 4 (l / 16) + r.

#pragma unroll
    for (int q = 0; q < 8; ++q) dma(q, 0, 0);
#pragma unroll
    for (int q = 0; q < 8; ++q) dma(q, 1, ktiles > 1 ? (uint32_t)TN_KB : 0u);
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");   // tile 0 (the first 8 of this wave's loads)
    __syncthreads();
    F8 fa, fb;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        rd8(fa, smem, 0, t);
        __builtin_amdgcn_sched_barrier(0);
    }

    for (int kt = 0; kt < ktiles; ++kt) {
        const int st = kt & 1;
        const uint8_t* base = smem + st * 2 * TM_SLICE;
        const uint8_t* next = smem + (st ^ 1) * 2 * TM_SLICE;
        const uint32_t kofs2 = (uint32_t)(kt + 2 < ktiles ? kt + 2 : ktiles - 1) * TN_KB;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            acc[q >> 2][q & 3] = Mfma16<T>::run(fa.b[q & 3], fa.a[q >> 2], acc[q >> 2][q & 3]);
            if (q & 1) rd8(fb, base, 1, q >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's part of tile kt + 1 landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            acc[q >> 2][q & 3] = Mfma16<T>::run(fb.b[q & 3], fb.a[q >> 2], acc[q >> 2][q & 3]);
            if (q & 1) dma(q >> 1, st, kofs2);
            else rd8(fa, next, 0, q >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- epilogue through LDS: each wave stages 32 rows x 64 columns at a time (rows padded to
    // 272 bytes, so the 16 rows one staging store writes start on distinct banks) in its own
    // 8.5 KB of the idle stage buffers, then reads whole 256-byte rows back, 4 per instruction.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    constexpr int EP_PITCH = 64 * 4 + 16;
    typedef Acc Acc4 __attribute__((ext_vector_type(4)));
    uint8_t* ep = smem + w * (32 * EP_PITCH);
    const int64_t row0 = (int64_t)tm * TM_TILE + wm * 64, col0 = (int64_t)tn * TM_TILE + wn * 64;
    Acc* cbase = C + row0 * ldc + col0;
    const int rc = lane & 15, rsub = lane >> 4;   // read-back: the lane's 16-byte chunk, row within 4
    int cols_in = 4;   // columns of this lane's 4-column group inside the matrix (RAGGED: 0..4)
    if constexpr (RAGGED) {
        const int64_t left = bnd.n - (col0 + 4 * rc);
        cols_in = left >= 4 ? 4 : (left > 0 ? (int)left : 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const Acc4 v = {acc[2 * i + ii][j][0], acc[2 * i + ii][j][1], acc[2 * i + ii][j][2],
                                acc[2 * i + ii][j][3]};
                *reinterpret_cast<Acc4*>(ep + (16 * ii + (lane & 15)) * EP_PITCH + (16 * j + 4 * (lane >> 4)) * 4) = v;
            }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's staged rows are in LDS
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int row = 4 * t + rsub;   // 0..31 of this half
            const Acc4 v = *reinterpret_cast<const Acc4*>(ep + row * EP_PITCH + rc * 16);
            Acc* dst = cbase + (int64_t)(32 * i + row) * ldc + 4 * rc;
            if (RAGGED && row0 + 32 * i + row >= bnd.m) continue;
            if (!RAGGED || (cols_in == 4 && bnd.cvec)) {
                __builtin_nontemporal_store(v, reinterpret_cast<Acc4*>(dst));
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k < cols_in) dst[k] = v[k];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // reads done before the next half overwrites
        __builtin_amdgcn_wave_barrier();
    }
}

template <typename T>
int mid_gemm_eligible(const void* A, const void* B, const void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc, bool ak, bool bk) {
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
    const size_t c_elem = sizeof(typename Mfma16<T>::acc_elem);
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
// column-major and B row-major within 6 % of these).  int8 with an M/N-contiguous operand, which the
// small-product kernel transposes by byte stores at about half its rate, keeps this kernel down to
// 64 tiles (TOP/s, A and B column-major: 2048^3 1167 / 627, 1024^2 x 8192 403 / 306, 1024^3 226 /
// 177; both M/N-contiguous 418 / 215 and 224 / 140).
bool mid_gemm_preferred(int64_t M, int64_t N, bool i8_mn) {
    const int64_t t128 = ((M + TM_TILE - 1) / TM_TILE) * ((N + TM_TILE - 1) / TM_TILE);
    const int64_t t256 = ((M + TN_TILE - 1) / TN_TILE) * ((N + TN_TILE - 1) / TN_TILE);
    return t128 >= (i8_mn ? 64 : 128) && t256 < 144;
}

template <typename T, bool AK, bool BK>
void launch_mid_layout(const T* A, const T* B, typename Mfma16<T>::acc_elem* C, int tiles_m, int tiles_n, int ktiles,
                       int64_t lda_b, int64_t ldb_b, int64_t ldc, const TnBounds& bnd, hipStream_t s, bool ragged) {
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    if (ragged)
        hipLaunchKernelGGL((gemm_mid_kernel<T, true, AK, BK>), grid, dim3(256), 0, s, A, B, C, tiles_m, tiles_n, ktiles,
                           lda_b, ldb_b, ldc, bnd);
    else
        hipLaunchKernelGGL((gemm_mid_kernel<T, false, AK, BK>), grid, dim3(256), 0, s, A, B, C, tiles_m, tiles_n, ktiles,
                           lda_b, ldb_b, ldc, bnd);
}

template <typename T>
int launch_gemm_mid(const T* A, const T* B, typename Mfma16<T>::acc_elem* C, int64_t M, int64_t N, int64_t K,
                    int64_t lda, int64_t ldb, int64_t ldc, hipStream_t s, bool ragged, bool ak, bool bk) {
    using Acc = typename Mfma16<T>::acc_elem;
    const int tiles_m = (int)((M + TM_TILE - 1) / TM_TILE), tiles_n = (int)((N + TM_TILE - 1) / TM_TILE);
    const int64_t ke = TN_KB / (int64_t)sizeof(T);
    const int ktiles = (int)((K + ke - 1) / ke);
    TnBounds bnd;
    bnd.m = M;
    bnd.n = N;
    bnd.kb = (int)(K * (int64_t)sizeof(T));
    bnd.cvec = ldc % 4 == 0 && aligned(C, 4 * sizeof(Acc));
    const int64_t lda_b = lda * (int64_t)sizeof(T), ldb_b = ldb * (int64_t)sizeof(T);
    if (!ak && !bk)
        launch_mid_layout<T, false, false>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, bnd, s, ragged);
    else if (!ak)
        launch_mid_layout<T, false, true>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, bnd, s, ragged);
    else if (!bk)
        launch_mid_layout<T, true, false>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, bnd, s, ragged);
    else
        launch_mid_layout<T, true, true>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, bnd, s, ragged);
    LAVA_LAUNCH_CHECK("gemm_mid_kernel");
    return LAVA_HIP_OK;
}

#define LAVA_MID_INST(T)                                                                                          \
    template int mid_gemm_eligible<T>(const void*, const void*, const void*, int64_t, int64_t, int64_t, int64_t, \
                                      int64_t, int64_t, bool, bool);                                              \
    template int launch_gemm_mid<T>(const T*, const T*, typename Mfma16<T>::acc_elem*, int64_t, int64_t, int64_t, \
                                    int64_t, int64_t, int64_t, hipStream_t, bool, bool, bool);
LAVA_MID_INST(f16)
LAVA_MID_INST(bf16)
LAVA_MID_INST(int8_t)
#undef LAVA_MID_INST

}  // namespace lava
