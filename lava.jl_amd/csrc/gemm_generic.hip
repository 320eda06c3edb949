// gemm_generic.hip -- GEMM kernels for every layout and any shape.
//
//  * gemm_staged_kernel: 64x64 output tile per workgroup of 4 wavefronts, one
//    K-slice of 64 bytes staged through LDS with bounds-predicated loads, so it
//    covers row- and column-major A and B and extents that are not tile
//    multiples (the clamp-to-zero of a TENSOR_CLAMP_CONSTANT load,
//    src/vocabulary/tensor.jl:46-51).  It is the fallback behind the fast TN
//    kernel and the path for small problems.
//  * gemm_small_kernel: the products too small to fill the chip with 256 x 256
//    tiles (16 or fewer of them, e.g. the 256^3 fp16 configuration): 64 x 64 tiles,
//    K in chunks of 512 bytes loaded with 16-byte loads, all in flight at once, the
//    next chunk arriving in registers while this one is multiplied.
//  * coopmat_tiles_kernel: the 16x16x16 subgroup-tile GEMM written in the
//    vocabulary exactly as docs/src/device.md:81-88 writes it -- one wavefront per
//    tile of C, fragments loaded straight from global memory.
#include <hip/hip_runtime.h>

#include <algorithm>
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

// 64 x 64 C tile per workgroup of 4 wavefronts (32 x 32 each: 2 x 2 MFMA 16x16 tiles).  K runs
// in chunks of 512 bytes.  A chunk of one operand is 64 rows (m or n) x 512 bytes = 2048 16-byte
// loads, 8 per thread, all issued before any is waited for; the next chunk's loads are in flight
// while this chunk is multiplied.  LDS layouts:
//  * a K-contiguous operand (A row-major, B column-major) is copied as loaded, [row][k], rows
//    padded to 528 bytes so that a fragment read (16 rows x one 16-byte chunk) is conflict-free;
//  * an M/N-contiguous 16-bit operand is copied as loaded too, [k][row] (128-byte rows padded to
//    144), and its fragments are read with two ds_read_b64_tr_b16 (4 k-values of one column per
//    lane each);
//  * an M/N-contiguous int8 operand is copied as loaded, [k][row] with 64-byte rows, chunk c of k
//    row k at slot c ^ F(k), F(k) = (k / 4 % 2) | 2 ((k / 16 + k / 32) % 2), and its fragments are
//    read with two ds_read_b64_tr_b8 (8 k-values of one column per lane each).  A 32-lane pass of
//    such a read covers 16 k rows (8 consecutive ones from each of two 16-lane groups, 16 or 32
//    apart) x one 16-byte column block; F gives the four rows of each k % 4 class distinct slots, so
//    the pass reads every bank once.
// Host conditions (small_gemm_fits): 16-byte aligned operands and leading dimensions, K a
// multiple of EV when an operand is K-contiguous, M (N) a multiple of EV when A (B) is M (N)-
// contiguous -- so every 16-byte chunk is wholly inside or wholly outside the matrix, and the
// outside ones read as zero.
// Split K: workgroup z multiplies K elements [z kspan, min(K, (z + 1) kspan)) and writes its
// product at C + z zstride (kspan a multiple of the 512-byte chunk; one split: kspan = K).
// U8 (int8 storage, no epilogue): the bytes are unsigned.  They are flipped to s = u - 128 (XOR
// 0x80) on their way into LDS, multiplied by the signed MFMA, and each C element gets
// 128 (RA + CB) + 16384 Kp added, RA / CB the sums of its row's / column's flipped bytes over the
// Kp k-values the workgroup multiplied (K padded to the 64-byte k-step: a padded byte reads 0,
// flips to -128 in both operands, and its terms cancel), all modulo 2^32.
template <typename T, bool AROW, bool BROW, typename OutT, bool EPI, bool U8 = false>
__global__ void __launch_bounds__(256) gemm_small_kernel(const T* __restrict__ A, const T* __restrict__ B,
                                                         OutT* __restrict__ C, int64_t M, int64_t N, int64_t K,
                                                         int64_t lda, int64_t ldb, int64_t ldc, Epilogue epi,
                                                         int64_t kspan, int64_t zstride) {
    static_assert(!U8 || (sizeof(T) == 1 && !EPI), "the unsigned form is int8 storage without an epilogue");
    using Acc = typename Mfma16<T>::acc_elem;
    using AccV = typename Mfma16<T>::acc_t;
    constexpr int EV = 16 / (int)sizeof(T);   // elements per 16-byte chunk
    constexpr int KC = 512 / (int)sizeof(T);  // elements of K per chunk
    constexpr int KE = Mfma16<T>::k;          // elements per MFMA k-step (64 bytes)
    constexpr int PITCH = 528;                // [row][k] layout: LDS bytes per row
    constexpr int PTR = 144;                  // [k][row] layout (16-bit types): LDS bytes per k
    constexpr int JR = 64 / EV;               // 16-byte chunks across the 64 rows of an M/N-contiguous chunk
    constexpr bool A_TR = !AROW;                      // A read through transposing LDS reads
    constexpr bool B_TR = BROW;
    constexpr int TR_BYTES = sizeof(T) == 2 ? KC * PTR : KC * 64;   // [k][row] staging of a transposed operand
    // each operand's staging sized for its own layout: int8 needs 2 x 33 KB at most, so two
    // workgroups share a CU
    __shared__ __attribute__((aligned(16))) uint8_t As[A_TR ? TR_BYTES : 64 * PITCH];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[B_TR ? TR_BYTES : 64 * PITCH];
    // the int8 [k][row] swizzle F(k)
    auto f8 = [](int k) __attribute__((always_inline)) { return ((k >> 2) & 1) | ((((k >> 4) ^ (k >> 5)) & 1) << 1); };

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
    const int wm = w >> 1, wn = w & 1;
    const int64_t kb = (int64_t)blockIdx.z * kspan, ke = min(K, kb + kspan);
    C += (int64_t)blockIdx.z * zstride;

    // 16-byte chunk i (of 8) of this thread for the K-chunk at k0 of operand X, whose rows r0 ..
    // r0 + 63 (m or n) are K-contiguous (kcont) or M/N-contiguous
    auto load = [&](const T* X, auto kcont, int64_t ld, int64_t r0, int64_t rows, int64_t k0, uint4* reg) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + 256 * i;
            int64_t rr, kk;
            const T* p;
            if constexpr (decltype(kcont)::value) {
                rr = r0 + (e >> 5);
                kk = k0 + (int64_t)EV * (e & 31);
                p = X + rr * ld + kk;
            } else {
                kk = k0 + e / JR;
                rr = r0 + (int64_t)EV * (e % JR);
                p = X + kk * ld + rr;
            }
            reg[i] = make_uint4(0, 0, 0, 0);
            if (rr < rows && kk < ke) reg[i] = *reinterpret_cast<const uint4*>(p);
        }
    };
    auto store = [&](uint8_t* S, auto kcont, auto tr, const uint4* reg) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + 256 * i;
            uint4 x = reg[i];
            if constexpr (U8) {
                x.x ^= 0x80808080u;
                x.y ^= 0x80808080u;
                x.z ^= 0x80808080u;
                x.w ^= 0x80808080u;
            }
            if constexpr (decltype(kcont)::value) {
                *reinterpret_cast<uint4*>(S + (e >> 5) * PITCH + 16 * (e & 31)) = x;
            } else if constexpr (sizeof(T) == 2) {
                *reinterpret_cast<uint4*>(S + (e / JR) * PTR + 16 * (e % JR)) = x;
            } else {
                const int k = e / JR, j = e % JR;   // k row, 16-byte column block
                *reinterpret_cast<uint4*>(S + k * 64 + 16 * (j ^ f8(k))) = x;
            }
        }
    };
    // fragment of rows rb .. rb + 15 at k-step ks: lane (r, g) = (lane % 16, lane / 16) holds
    // row rb + r, k 8 g .. 8 g + 7 of the step
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    typedef int tr8_v2i __attribute__((ext_vector_type(2)));
    auto frag = [&](const uint8_t* S, auto tr, int rb, int ks) -> uint4 {
        if constexpr (decltype(tr)::value && sizeof(T) == 1) {
            // source lane s of group g points at k row 16 g + s / 2 (+ 8) of the step, byte 8 (s % 2)
            // of column block rb / 16: output lane i gets 8 k-values of column rb + i per read
            const int g = lane >> 4, s2 = lane & 15;
            const int k = ks * KE + 16 * g + (s2 >> 1);   // bit 3 clear: k + 8 has the same F
            const uint8_t* p0 = S + k * 64 + 16 * ((rb >> 4) ^ f8(k)) + 8 * (s2 & 1);
            const tr8_v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (__attribute__((address_space(3))) tr8_v2i*)(const __attribute__((address_space(3))) uint8_t*)(p0));
            const tr8_v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (__attribute__((address_space(3))) tr8_v2i*)(const __attribute__((address_space(3))) uint8_t*)(p0 + 8 * 64));
            return make_uint4((uint32_t)lo.x, (uint32_t)lo.y, (uint32_t)hi.x, (uint32_t)hi.y);
        } else if constexpr (decltype(tr)::value) {
            // source lane (jj, q) = ((lane % 16) / 4, lane % 4) of group g points at k row
            // 8 g + jj (+ 4), rows rb + 4 q .. + 3: output lane r gets 4 k-values of row rb + r
            const int g = lane >> 4, jj = (lane & 15) >> 2, q = lane & 3;
            const uint8_t* p0 = S + (ks * KE + 8 * g + jj) * PTR + 2 * (rb + 4 * q);
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(const __attribute__((address_space(3))) uint8_t*)(p0));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(const __attribute__((address_space(3))) uint8_t*)(p0 + 4 * PTR));
            return __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        } else {
            return *reinterpret_cast<const uint4*>(S + (rb + (lane & 15)) * PITCH + ks * 64 + (lane >> 4) * 16);
        }
    };
    typedef std::integral_constant<bool, AROW> AK;    // A row-major: K-contiguous
    typedef std::integral_constant<bool, !BROW> BK;   // B column-major: K-contiguous
    typedef std::integral_constant<bool, A_TR> ATR;
    typedef std::integral_constant<bool, B_TR> BTR;

    AccV acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = AccV{0, 0, 0, 0};
    // U8: this lane's sums of the flipped bytes of its fragment rows (A) and columns (B), and the
    // k-steps multiplied
    uint32_t usa[2] = {0u, 0u}, usb[2] = {0u, 0u};
    int64_t usteps = 0;
    auto bytesum = [](uint4 v, uint32_t acc) __attribute__((always_inline)) {
        int s = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, (int)acc, false);
        s = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, s, false);
        s = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, s, false);
        return (uint32_t)__builtin_amdgcn_sdot4((int)v.w, 0x01010101, s, false);
    };
    uint4 ra[8], rb[8];
    load(A, AK{}, lda, m0, M, kb, ra);
    load(B, BK{}, ldb, n0, N, kb, rb);
    for (int64_t k0 = kb; k0 < ke; k0 += KC) {
        store(As, AK{}, ATR{}, ra);
        store(Bs, BK{}, BTR{}, rb);
        __syncthreads();
        if (k0 + KC < ke) {   // the next chunk, in flight during this one's MFMAs
            load(A, AK{}, lda, m0, M, k0 + KC, ra);
            load(B, BK{}, ldb, n0, N, k0 + KC, rb);
        }
        const int64_t nks = min((int64_t)(KC / KE), (ke - k0 + KE - 1) / KE);
        if constexpr (U8) usteps += nks;
#pragma unroll
        for (int ks = 0; ks < KC / KE; ++ks) {
            if (ks < nks) {
                uint4 af[2], bf[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    af[t] = frag(As, ATR{}, wm * 32 + t * 16, ks);
                    bf[t] = frag(Bs, BTR{}, wn * 32 + t * 16, ks);
                }
                if constexpr (U8) {
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        usa[t] = bytesum(af[t], usa[t]);
                        usb[t] = bytesum(bf[t], usb[t]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[i][j] = Mfma16<T>::run(af[i], bf[j], acc[i][j]);
            }
        }
        __syncthreads();
    }
    if constexpr (U8) {
        // lane (r, g) summed fragment row / column r over k slice g: add the four slices, so every
        // lane holds the full sum of row (column) lane % 16 of each fragment
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            usa[t] += (uint32_t)__shfl_xor((int)usa[t], 16);
            usa[t] += (uint32_t)__shfl_xor((int)usa[t], 32);
            usb[t] += (uint32_t)__shfl_xor((int)usb[t], 16);
            usb[t] += (uint32_t)__shfl_xor((int)usb[t], 32);
        }
        const uint32_t kconst = 16384u * (uint32_t)(usteps * KE);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t rsum = (uint32_t)__shfl((int)usa[i], 4 * (lane >> 4) + q);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j][q] = (Acc)((uint32_t)acc[i][j][q] + 128u * (rsum + usb[j]) + kconst);
            }
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

// The split-K sum: C[m][n] = the splits' partial products P[z][m][n] (row-major, M x N each)
// added in split order, so a result does not depend on the order the workgroups ran in; int32
// partials add modulo 2^32, as the MFMA accumulates.  VEC (N a multiple of 4): each thread sums 4
// adjacent columns through 16-byte loads (P is 16-byte aligned).  Grid (ceil(N / (256 VEC)), M).
template <typename Acc, int VEC>
__global__ void __launch_bounds__(256) splitk_sum_kernel(const Acc* __restrict__ P, Acc* __restrict__ C, int64_t M,
                                                         int64_t N, int64_t ldc, int splits) {
    const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC, m = blockIdx.y;
    if (n >= N) return;
    const int64_t e = m * N + n, mn = M * N;
    auto add = [](Acc x, Acc y) -> Acc {
        if constexpr (std::is_same<Acc, int32_t>::value)
            return (int32_t)((uint32_t)x + (uint32_t)y);
        else
            return x + y;
    };
    if constexpr (VEC == 4) {
        using V = typename std::conditional<std::is_same<Acc, int32_t>::value, int4, float4>::type;
        V sum = *reinterpret_cast<const V*>(P + e);
        for (int z = 1; z < splits; ++z) {
            const V p = *reinterpret_cast<const V*>(P + z * mn + e);
            sum.x = add(sum.x, p.x);
            sum.y = add(sum.y, p.y);
            sum.z = add(sum.z, p.z);
            sum.w = add(sum.w, p.w);
        }
        Acc* c = C + m * ldc + n;
        c[0] = sum.x;
        c[1] = sum.y;
        c[2] = sum.z;
        c[3] = sum.w;
    } else {
        Acc sum = P[e];
        for (int z = 1; z < splits; ++z) sum = add(sum, P[z * mn + e]);
        C[m * ldc + n] = sum;
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

template <typename T>
bool small_gemm_preferred(int64_t M, int64_t N, int64_t) {
    const int64_t tiles256 = ((M + 255) / 256) * ((N + 255) / 256);
    if (tiles256 <= SMALL_GEMM_MAX_TILES) return true;
    // Rate estimates (measured on shape lists): the tile kernel ~1500 TFLOP/s (bf16; int8 ~3000
    // TOP/s) times the share of the 256 CUs its tiles occupy times the useful share of the tile
    // area, the small kernel ~450 (int8 ~800, two workgroups per CU) times the share of 512
    // workgroups its 64 x 64 tiles fill.  E.g. bf16 64 x 14336 x 4096: 94 -> 234 TFLOP/s; 1536^2
    // x 8192: 275 -> 342; 2048 x 4096 x 4096 stays on the tile kernel (898 against 494); int8
    // (tile kernel against small kernel, TOP/s): 64 x 14336 x 4096 166 / 383, 128 x 28672 x 8192
    // 727 / 755, 2048^3 653 / 681, 1536^2 x 8192 515 / 637 take the small kernel, 2048 x 4096 x
    // 4096 (1558 / 916) the tile kernel.  An M/N-contiguous operand (Julia's column-major default) is
    // read through transposing LDS reads on every kernel, at about the K-contiguous rate (int8 64 x
    // 14336 x 4096 with A column-major 391 TOP/s against 390; 2048^3 621 against 694).
    const double tile_rate = sizeof(T) == 1 ? 3000.0 : 1500.0;
    const double small_rate = sizeof(T) == 1 ? 800.0 : 450.0;
    const int64_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
    const double occ256 = tiles256 >= 256 ? 1.0 : (double)tiles256 / 256.0;
    const double useful = (double)M * (double)N / ((double)tiles256 * 65536.0);
    const double occ64 = tiles64 >= 512 ? 1.0 : (double)tiles64 / 512.0;
    return tile_rate * occ256 * useful < small_rate * occ64;
}

template <typename T>
bool small_gemm_fits(const void* A, const void* B, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, bool arow,
                     bool brow) {
    constexpr int64_t EV = 16 / (int64_t)sizeof(T);
    // the launch puts M / 64 in gridDim.y (at most 65535)
    if ((M + 63) / 64 > 65535 || (N + 63) / 64 > 0x7fffffff) return false;
    return aligned(A, 16) && aligned(B, 16) && lda % EV == 0 && ldb % EV == 0 &&
           ((arow || !brow) ? K % EV == 0 : true) && (arow || M % EV == 0) && (!brow || N % EV == 0);
}
#define LAVA_SMALL_RULE_INST(T)                                                                                      \
    template bool small_gemm_preferred<T>(int64_t, int64_t, int64_t);                                           \
    template bool small_gemm_fits<T>(const void*, const void*, int64_t, int64_t, int64_t, int64_t, int64_t, bool, bool);
LAVA_SMALL_RULE_INST(f16)
LAVA_SMALL_RULE_INST(bf16)
LAVA_SMALL_RULE_INST(int8_t)
#undef LAVA_SMALL_RULE_INST

namespace {
template <typename T, typename OutT, bool EPI, bool U8 = false>
int launch_small_grid(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                      int64_t ldc, bool arow, bool brow, hipStream_t s, const Epilogue& epi, int splits,
                      int64_t kspan, int64_t zstride) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64), (unsigned)splits);
    if (arow && brow)
        hipLaunchKernelGGL((gemm_small_kernel<T, true, true, OutT, EPI, U8>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi, kspan, zstride);
    else if (arow)
        hipLaunchKernelGGL((gemm_small_kernel<T, true, false, OutT, EPI, U8>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi, kspan, zstride);
    else if (brow)
        hipLaunchKernelGGL((gemm_small_kernel<T, false, true, OutT, EPI, U8>), grid, dim3(256), 0, s, A, B, C, M, N, K,
                           lda, ldb, ldc, epi, kspan, zstride);
    else
        hipLaunchKernelGGL((gemm_small_kernel<T, false, false, OutT, EPI, U8>), grid, dim3(256), 0, s, A, B, C, M, N,
                           K, lda, ldb, ldc, epi, kspan, zstride);
    LAVA_LAUNCH_CHECK(U8 ? "gemm_small_kernel<u8>" : "gemm_small_kernel");
    return LAVA_HIP_OK;
}
}  // namespace

int launch_gemm_small_u8(const int8_t* A, const int8_t* B, int32_t* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, bool arow, bool brow, hipStream_t s) {
    return launch_small_grid<int8_t, int32_t, false, true>(A, B, C, M, N, K, lda, ldb, ldc, arow, brow, s, Epilogue{},
                                                           1, K > 0 ? K : 1, 0);
}

template <typename T, typename OutT, bool EPI>
int launch_gemm_small(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                      int64_t ldc, bool arow, bool brow, hipStream_t s, const Epilogue& epi) {
    return launch_small_grid<T, OutT, EPI>(A, B, C, M, N, K, lda, ldb, ldc, arow, brow, s, epi, 1, K > 0 ? K : 1, 0);
}

template <typename T>
SmallSplit small_gemm_splits(int64_t M, int64_t N, int64_t K) {
    constexpr int64_t KC = 512 / (int64_t)sizeof(T);   // the kernel's K chunk
    const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
    const int64_t chunks = (K + KC - 1) / KC;
    SmallSplit r;
    // Measured (bf16, one box): 512^2 x 4096 (64 tiles, 16 chunks) 73 -> 124 TFLOP/s, 1024^2 x
    // 8192 (256 tiles, 32 chunks) 323 -> 379, 64 x 14336 x 4096 232 -> 259, while 1024^3 (256
    // tiles, 4 chunks) fell 186 -> 128: the partial products' round trip and the second launch
    // outweigh a short K, more so where the tiles already occupy half the chip.
    if (tiles > 256 || chunks < (tiles > 128 ? 16 : 8)) return r;
    int64_t want = std::min<int64_t>(std::min<int64_t>(chunks / 2, 512 / tiles), SMALL_GEMM_MAX_SPLITS);
    if (want < 2) return r;
    const int64_t per = (chunks + want - 1) / want;   // chunks per split
    r.splits = (int)((chunks + per - 1) / per);
    r.kspan = per * KC;
    return r;
}

template <typename T>
size_t small_splitk_bytes(int64_t M, int64_t N, const SmallSplit& sp) {
    return STREAM_WS_RESERVED + (size_t)M * (size_t)N * sizeof(typename Mfma16<T>::acc_elem) * (size_t)sp.splits;
}
template size_t small_splitk_bytes<f16>(int64_t, int64_t, const SmallSplit&);
template size_t small_splitk_bytes<bf16>(int64_t, int64_t, const SmallSplit&);
template size_t small_splitk_bytes<int8_t>(int64_t, int64_t, const SmallSplit&);

template <typename T, bool U8>
int launch_gemm_small_splitk(const T* A, const T* B, typename Mfma16<T>::acc_elem* C, int64_t M, int64_t N, int64_t K,
                             int64_t lda, int64_t ldb, int64_t ldc, bool arow, bool brow, void* stream,
                             const SmallSplit& sp) {
    using Acc = typename Mfma16<T>::acc_elem;
    hipStream_t s = as_stream(stream);
    return with_stream_workspace(small_splitk_bytes<T>(M, N, sp), stream, [&](void* ws) {
        Acc* P = reinterpret_cast<Acc*>(static_cast<uint8_t*>(ws) + STREAM_WS_RESERVED);
        // unsigned: each split's partial carries its own correction, so the wrapped sum of the
        // partials is the product
        int rc = launch_small_grid<T, Acc, false, U8>(A, B, P, M, N, K, lda, ldb, N, arow, brow, s, Epilogue{},
                                                     sp.splits, sp.kspan, M * N);
        if (rc != LAVA_HIP_OK) return rc;
        if (N % 4 == 0)
            hipLaunchKernelGGL((splitk_sum_kernel<Acc, 4>), dim3((unsigned)((N + 1023) / 1024), (unsigned)M), dim3(256),
                               0, s, P, C, M, N, ldc, sp.splits);
        else
            hipLaunchKernelGGL((splitk_sum_kernel<Acc, 1>), dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256),
                               0, s, P, C, M, N, ldc, sp.splits);
        LAVA_LAUNCH_CHECK("splitk_sum_kernel");
        return LAVA_HIP_OK;
    });
}
template SmallSplit small_gemm_splits<f16>(int64_t, int64_t, int64_t);
template SmallSplit small_gemm_splits<bf16>(int64_t, int64_t, int64_t);
template SmallSplit small_gemm_splits<int8_t>(int64_t, int64_t, int64_t);
template int launch_gemm_small_splitk<f16, false>(const f16*, const f16*, float*, int64_t, int64_t, int64_t, int64_t,
                                                  int64_t, int64_t, bool, bool, void*, const SmallSplit&);
template int launch_gemm_small_splitk<bf16, false>(const bf16*, const bf16*, float*, int64_t, int64_t, int64_t,
                                                   int64_t, int64_t, int64_t, bool, bool, void*, const SmallSplit&);
template int launch_gemm_small_splitk<int8_t, false>(const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t,
                                                     int64_t, int64_t, int64_t, bool, bool, void*, const SmallSplit&);
template int launch_gemm_small_splitk<int8_t, true>(const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t,
                                                    int64_t, int64_t, int64_t, bool, bool, void*, const SmallSplit&);

#define LAVA_STAGED_INST(T, O, E)                                                                              \
    template int launch_gemm_staged<T, O, E>(const T*, const T*, O*, int64_t, int64_t, int64_t, int64_t, int64_t, \
                                             int64_t, bool, bool, hipStream_t, const Epilogue&);                  \
    template int launch_gemm_small<T, O, E>(const T*, const T*, O*, int64_t, int64_t, int64_t, int64_t, int64_t,  \
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

// Unsigned bytes, any shape and layout: one thread per element of C, uint32 sums (wrapping, as
// the cooperative-matrix integer accumulator does).
__global__ void __launch_bounds__(256) gemm_u8_generic_kernel(const uint8_t* __restrict__ A,
                                                              const uint8_t* __restrict__ B, uint32_t* __restrict__ C,
                                                              int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                                              int64_t ldc, uint32_t layout) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * N) return;
    const bool arow = layout & 1u, brow = layout & 2u, crow = layout & 4u;
    const int64_t m = idx / N, n = idx % N;
    uint32_t acc = 0;
    for (int64_t k = 0; k < K; ++k)
        acc += (uint32_t)A[arow ? m * lda + k : k * lda + m] * (uint32_t)B[brow ? k * ldb + n : n * ldb + k];
    C[crow ? m * ldc + n : n * ldc + m] = acc;
}

int launch_gemm_u8_generic(const uint8_t* A, const uint8_t* B, uint32_t* C, int64_t M, int64_t N, int64_t K,
                           int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout, hipStream_t s) {
    hipLaunchKernelGGL(gemm_u8_generic_kernel, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, s, A, B, C, M, N,
                       K, lda, ldb, ldc, layout);
    LAVA_LAUNCH_CHECK("gemm_u8_generic_kernel");
    return LAVA_HIP_OK;
}

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
