// gemm_mid_kernel.hpp -- the mid-size GEMM kernel (gemm_mid_kernel) and its launcher (internal):
// 128 x 128 tiles of C, for products whose 256 x 256 tiles would leave most of the 256 CUs idle
// (2048^3: 64 of them, against 256 tiles of 128 x 128) and that the 64 x 64 small-product kernel runs
// well below the matrix cores' rate.  f16, bf16 or int8, each operand K-contiguous (A row-major, B
// column-major) or M/N-contiguous; fp32 / int32 output, or for f16 / bf16 the fused epilogue (bias,
// residual, activation, narrowed to fp32 / f16 / bf16), or for unsigned bytes the uint32 product.
// The staging is the tile kernel's at 128 rows (gemm_tn_kernel.hpp: TnSide<T, true, 128>, LDS-DMA of 128 bytes of K per m or n row, chunk ^ row %
// 8; TnSide<T, false, 128>, 128 bytes of K as rows of 128 m or n, read back transposed) on a quarter
// of its LDS, so that two workgroups share a CU and their wavefronts interleave on each SIMD:
//  * 4 wavefronts, each a 64 x 64 sub-tile = 4 x 4 16x16 accumulators (64 registers per lane);
//  * K advances 128 bytes per k-tile: A and B slices of 16 KB each, double-buffered (64 KB);
//  * per k-tile, as in the tile kernel: 16 MFMAs of k-step 0 with k-step 1's 8 fragment reads,
//    the barrier (this wavefront's DMAs of the next tile landed), 16 MFMAs of k-step 1 with the
//    next tile's k-step 0 reads and the 8 DMAs of the tile after next;
//  * the epilogue stages 32 rows x 64 columns per wavefront at a time through LDS and stores whole
//    row runs (4 rows per instruction), nontemporal; with the fused epilogue the lane's bias and
//    residual values of a half are requested before its staging, as in the tile kernel.
// The plain instances live in gemm_mid.hip, the fused-epilogue and unsigned ones in gemm_mid_ex.hip.
#pragma once
#include "gemm_tn_kernel.hpp"

namespace lava {

constexpr int TM_TILE = 128;
constexpr int TM_SLICE = TM_TILE * TN_KB;   // 16 KB

// U8 (T = int8_t storage holding unsigned bytes, int32 C holding the uint32 product): the tile
// kernel's identity (gemm_tn_kernel.hpp) -- signed MFMAs on the bytes flipped by 128, C = A_s B_s +
// 128 (RA[m] + CB[n]) + 16384 Kp modulo 2^32 with RA, CB the row and column sums of the flipped
// bytes and Kp the k positions accumulated, zero padding included.
template <typename T, typename OutT, bool EPI, bool RAGGED, bool AK, bool BK, bool U8 = false>
__global__ void __launch_bounds__(256, 2)
    gemm_mid_kernel(const T* __restrict__ A, const T* __restrict__ B, OutT* __restrict__ C, int tiles_m, int tiles_n,
                    int ktiles, int64_t lda_b, int64_t ldb_b, int64_t ldc, Epilogue epi, TnBounds bnd) {
    using AccV = typename Mfma16<T>::acc_t;
    typedef typename Mfma16<T>::acc_elem Acc;
    static_assert(EPI || std::is_same<OutT, Acc>::value, "a plain product writes the accumulator type");
    static_assert(!U8 || (std::is_same<T, int8_t>::value && !EPI), "U8: bytes in int8_t storage, plain int32 output");
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
    // U8: signed-byte sums of this wavefront's A rows (ra[i]: row 16 i + lane % 16 of its 64) and
    // B columns (rb[j]), over the k bytes of this lane's 16-lane group
    int32_t ra[4], rb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = rb[i] = 0;
    auto flip = [&](uint4& v, int32_t& sum) __attribute__((always_inline)) {
        v.x ^= 0x80808080u;
        v.y ^= 0x80808080u;
        v.z ^= 0x80808080u;
        v.w ^= 0x80808080u;
        sum = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, sum, false);
        sum = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, sum, false);
        sum = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, sum, false);
        sum = __builtin_amdgcn_sdot4((int)v.w, 0x01010101, sum, false);
    };
    // fragment t in read order (a[0], b[0..3], a[1..3]).  Each is flipped two reads after its own
    // read was issued, before its first MFMA; the last two of a k-step (a[2], a[3], first used by
    // MFMAs 8 and 12) are flipped at MFMAs 2 and 6 of the next half.  Fragments read past the last
    // k-tile are never flipped, so they do not enter the sums.
    auto flip_t = [&](F8& f, int t) __attribute__((always_inline)) {
        if constexpr (U8) {
            if (t == 0) flip(f.a[0], ra[0]);
            else if (t <= 4) flip(f.b[t - 1], rb[t - 1]);
            else flip(f.a[t - 4], ra[t - 4]);
        }
    };
#pragma unroll
    for (int t = 0; t < 8; ++t) flip_t(fa, t);

    for (int kt = 0; kt < ktiles; ++kt) {
        const int st = kt & 1;
        const uint8_t* base = smem + st * 2 * TM_SLICE;
        const uint8_t* next = smem + (st ^ 1) * 2 * TM_SLICE;
        const uint32_t kofs2 = (uint32_t)(kt + 2 < ktiles ? kt + 2 : ktiles - 1) * TN_KB;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            acc[q >> 2][q & 3] = Mfma16<T>::run(fa.b[q & 3], fa.a[q >> 2], acc[q >> 2][q & 3]);
            if (q & 1) rd8(fb, base, 1, q >> 1);
            if ((q == 2 || q == 6) && kt > 0) flip_t(fa, 6 + (q >> 2));
            if ((q & 1) && q >= 5) flip_t(fb, (q >> 1) - 2);
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
            if (q == 2 || q == 6) flip_t(fb, 6 + (q >> 2));
            if (!(q & 1) && q >= 4 && kt + 1 < ktiles) flip_t(fa, (q >> 1) - 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- epilogue through LDS: each wave stages 32 rows x 64 columns at a time (rows padded to
    // 272 bytes, so the 16 rows one staging store writes start on distinct banks) in its own
    // 8.5 KB of the idle stage buffers, then reads whole 256-byte rows back, 4 per instruction.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if constexpr (U8) {
        // full sums: the four 16-lane groups hold the four 16-byte quarters of every k-step
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ra[i] += __shfl_xor(ra[i], 16, 64);
            ra[i] += __shfl_xor(ra[i], 32, 64);
            rb[i] += __shfl_xor(rb[i], 16, 64);
            rb[i] += __shfl_xor(rb[i], 32, 64);
        }
        // acc[i][j] register r: row 16 i + lane % 16 (this lane's ra[i]), column 16 j + 4 (lane / 16) + r
        // (rb[j] of lane 4 (lane / 16) + r)
        const uint32_t kconst = 16384u * (uint32_t)ktiles * (uint32_t)TN_KB;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t cb[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) cb[r] = (uint32_t)__shfl(rb[j], 4 * (lane >> 4) + r, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[i][j][r] = (int32_t)((uint32_t)acc[i][j][r] + 128u * ((uint32_t)ra[i] + cb[r]) + kconst);
        }
    }
    constexpr int EP_PITCH = 64 * 4 + 16;
    typedef Acc Acc4 __attribute__((ext_vector_type(4)));
    typedef float F4 __attribute__((ext_vector_type(4)));
    uint8_t* ep = smem + w * (32 * EP_PITCH);
    const int64_t row0 = (int64_t)tm * TM_TILE + wm * 64, col0 = (int64_t)tn * TM_TILE + wn * 64;
    OutT* cbase = C + row0 * ldc + col0;
    const int rc = lane & 15, rsub = lane >> 4;   // read-back: the lane's 16-byte chunk, row within 4
    int cols_in = 4;   // columns of this lane's 4-column group inside the matrix (RAGGED: 0..4)
    if constexpr (RAGGED) {
        const int64_t left = bnd.n - (col0 + 4 * rc);
        cols_in = left >= 4 ? 4 : (left > 0 ? (int)left : 0);
    }
    // one half (32 rows) at a time; i is a template constant so that acc stays in registers
    auto half = [&](auto itag) {
        constexpr int i = decltype(itag)::value;
        // the fused epilogue's terms for the 8 rows x 4 columns this lane stores, requested before
        // the staging so that their latency overlaps it
        F4 rin[EPI ? 8 : 1];
        float bin[EPI ? 8 : 1];
        F4 bcol = {0.f, 0.f, 0.f, 0.f};
        if constexpr (EPI) {
            const int64_t n = col0 + 4 * rc;
            // 4 floats at p, or those of them inside the matrix (columns < N)
            auto ld4 = [&](const float* p) {
                if (epi.vec4 && cols_in == 4) return *reinterpret_cast<const F4*>(p);
                F4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k < cols_in) r[k] = p[k];
                return r;
            };
            if (epi.bias && epi.bias_on_cols) bcol = ld4(epi.bias + n);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int64_t m = row0 + 32 * i + 4 * t + rsub;
                rin[t] = F4{0.f, 0.f, 0.f, 0.f};
                bin[t] = 0.f;
                if (RAGGED && m >= bnd.m) continue;
                if (epi.residual) rin[t] = ld4(epi.residual + m * epi.ldr + n);
                if (epi.bias && !epi.bias_on_cols) bin[t] = epi.bias[m];
            }
        }
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
        auto store_rows = [&](auto acttag) {
            constexpr int ACT = decltype(acttag)::value;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int row = 4 * t + rsub;   // 0..31 of this half
                const Acc4 v = *reinterpret_cast<const Acc4*>(ep + row * EP_PITCH + rc * 16);
                OutT* dst = cbase + (int64_t)(32 * i + row) * ldc + 4 * rc;
                if (RAGGED && row0 + 32 * i + row >= bnd.m) continue;
                if constexpr (!EPI) {
                    if (!RAGGED || (cols_in == 4 && bnd.cvec)) {
                        __builtin_nontemporal_store(v, reinterpret_cast<Acc4*>(dst));
                    } else {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (k < cols_in) dst[k] = v[k];
                    }
                } else {
                    // the fused epilogue on 4 consecutive columns of one row, narrowed (RNE) to D's type
                    typedef OutT Out4 __attribute__((ext_vector_type(4)));
                    Out4 o;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        // the same fp32 sums as epi_apply: (bias + residual), then acc + that
                        const float x = epi_act_c<ACT>((float)v[k] + ((bin[t] + bcol[k]) + rin[t][k]));
                        o[k] = narrow<OutT>(x);
                    }
                    if (!RAGGED || (cols_in == 4 && bnd.cvec)) {
                        __builtin_nontemporal_store(o, reinterpret_cast<Out4*>(dst));
                    } else {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (k < cols_in) dst[k] = o[k];
                    }
                }
            }
        };
        if constexpr (EPI) {
            switch (epi.act) {   // uniform: one branch per half, none per element
            case EPI_RELU: store_rows(std::integral_constant<int, EPI_RELU>{}); break;
            case EPI_GELU_TANH: store_rows(std::integral_constant<int, EPI_GELU_TANH>{}); break;
            case EPI_GELU_ERF: store_rows(std::integral_constant<int, EPI_GELU_ERF>{}); break;
            default: store_rows(std::integral_constant<int, EPI_NONE>{}); break;
            }
        } else {
            store_rows(std::integral_constant<int, EPI_NONE>{});
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // reads done before the next half overwrites
        __builtin_amdgcn_wave_barrier();
    };
    half(std::integral_constant<int, 0>{});
    half(std::integral_constant<int, 1>{});
}

template <typename T, typename OutT, bool EPI, bool AK, bool BK, bool U8>
void launch_mid_layout(const T* A, const T* B, OutT* C, int tiles_m, int tiles_n, int ktiles, int64_t lda_b,
                       int64_t ldb_b, int64_t ldc, const Epilogue& epi, const TnBounds& bnd, hipStream_t s,
                       bool ragged) {
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    if (ragged)
        hipLaunchKernelGGL((gemm_mid_kernel<T, OutT, EPI, true, AK, BK, U8>), grid, dim3(256), 0, s, A, B, C, tiles_m,
                           tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd);
    else
        hipLaunchKernelGGL((gemm_mid_kernel<T, OutT, EPI, false, AK, BK, U8>), grid, dim3(256), 0, s, A, B, C, tiles_m,
                           tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd);
}

template <typename T, typename OutT, bool EPI, bool U8>
int launch_gemm_mid(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                    int64_t ldc, hipStream_t s, const Epilogue& epi, bool ragged, bool ak, bool bk) {
    const int tiles_m = (int)((M + TM_TILE - 1) / TM_TILE), tiles_n = (int)((N + TM_TILE - 1) / TM_TILE);
    const int64_t ke = TN_KB / (int64_t)sizeof(T);
    const int ktiles = (int)((K + ke - 1) / ke);
    TnBounds bnd;
    bnd.m = M;
    bnd.n = N;
    bnd.kb = (int)(K * (int64_t)sizeof(T));
    bnd.cvec = ldc % 4 == 0 && aligned(C, 4 * sizeof(OutT));
    const int64_t lda_b = lda * (int64_t)sizeof(T), ldb_b = ldb * (int64_t)sizeof(T);
    if (!ak && !bk)
        launch_mid_layout<T, OutT, EPI, false, false, U8>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd,
                                                      s, ragged);
    else if (!ak)
        launch_mid_layout<T, OutT, EPI, false, true, U8>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd, s,
                                                     ragged);
    else if (!bk)
        launch_mid_layout<T, OutT, EPI, true, false, U8>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd, s,
                                                     ragged);
    else
        launch_mid_layout<T, OutT, EPI, true, true, U8>(A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd, s,
                                                    ragged);
    LAVA_LAUNCH_CHECK("gemm_mid_kernel");
    return LAVA_HIP_OK;
}

#define LAVA_MID_LAUNCH_INST(T, O, E, U)                                                                          \
    template int launch_gemm_mid<T, O, E, U>(const T*, const T*, O*, int64_t, int64_t, int64_t, int64_t, int64_t,  \
                                             int64_t, hipStream_t, const Epilogue&, bool, bool, bool);

}  // namespace lava
