// gemm_w8a16.hip -- decode-shape GEMM with int8 weights and a per-column scale.
//
// Lava writes this as a coopmat GEMM whose epilogue is a per-element callback
// carrying the scale pointer in `extras` (src/device/coopmat_intrinsics.jl:535-628,
// 569-572): Y[r, c] = s[c] * sum_k X[r, k] W[k, c].  At M = 16 the product is
// bound by reading W once from HBM (58.7 MB at the headline shape), so the kernel
// is a weight stream:
//
//  * a wavefront owns 128 columns and a 32-row slice of K per step: lane (q, g)
//    = (lane % 16, lane / 16) loads 8 bytes (columns 8q .. 8q + 7) of the 8 rows
//    8g .. 8g + 7 -- 16 lanes cover one 128-byte row segment;
//  * those 64 bytes are 8 columns x 8 k-values; column t of them is lane q's
//    column of MFMA tile t (tile t = columns {8q + t}), k-values in lane group g:
//    exactly the B operand of v_mfma_f32_16x16x32_f16, after an in-register byte
//    transpose (v_perm_b32) and an exact int8 -> fp16 conversion
//    (0x6400 | (w ^ 0x80) is the fp16 value 1152 + w; subtract 1152);
//  * X (16 x 32 per step, fp16) is the A operand, read straight from global/L2;
//  * 8 wavefronts per workgroup split the workgroup's K range and reduce through
//    LDS; to occupy every CU (N / 128 column blocks alone leave most of them idle)
//    `splits` workgroups split K further.  Each writes its (scaled) partial block to a
//    workspace and counts itself in at a per-block arrival counter; the last of the
//    `splits` workgroups adds the partial blocks in split order (fixed: deterministic)
//    and writes Y, and resets the counter for the next call -- one launch, no second
//    reduction kernel;
//  * the weight rows of up to W8_DEPTH K steps are in flight ahead of the MFMAs;
//  * the scale multiply is the fused per-element epilogue, applied to every partial.
#include <hip/hip_runtime.h>

#include <functional>
#include <map>
#include <mutex>
#include <set>
#include <type_traits>
#include <vector>

#include "lava_coopmat.hpp"
#include "lava_hip_internal.hpp"
#include "lds_dma.hpp"

namespace lava {

constexpr int W8_COLS = 128;   // columns per workgroup
constexpr int W8_KSTEP = 32;   // k per MFMA step
constexpr int W8_WAVES = 8;
constexpr int W8_DEPTH = 4;   // K steps of weights in flight per wavefront

__device__ __forceinline__ uint32_t w8_pair(uint32_t lo_row, uint32_t hi_row, int byte) {
    // [lo_row.byte, 0, hi_row.byte, 0] -> two fp16 values 1152 + w, then subtract 1152
    const uint32_t sel = (uint32_t)byte | 0x0c00u | ((uint32_t)(byte + 4) << 16) | 0x0c000000u;
    return __builtin_amdgcn_perm(hi_row, lo_row, sel) ^ 0x64806480u;
}

// The dequant callback f(r, c, e, s, base) = e * s[base + STRIDE c]: tile column c of a
// kernel whose tile t holds the columns base = n0 + t, n0 + t + STRIDE, ...
template <int STRIDE>
struct ScaleStrided {
    __device__ float operator()(uint32_t, uint32_t col, float e, const f16* s, uint32_t base) const {
        return e * (float)s[base + STRIDE * col];
    }
};
// The same with the columns at or past n (a ragged last column block) giving zero; the load is
// unconditional, from a clamped index, so that the loads of a fragment stay in flight together
// (a predicated load waits for each in turn).
template <int STRIDE>
struct ScaleStridedBounded {
    __device__ float operator()(uint32_t, uint32_t col, float e, const f16* s, uint32_t base, uint32_t n) const {
        const uint32_t c = base + STRIDE * col;
        const float sc = (float)s[c < n ? c : n - 1];
        return c < n ? e * sc : 0.f;
    }
};

// Wavefront gw = split * W8_WAVES + w takes the 32-row steps [gw ks, min((gw + 1) ks,
// total_steps)) of K.  KSTEPS > 0: the host guarantees exactly KSTEPS each, fully
// unrolled; KSTEPS == 0: any count (zero included), in unrolled groups of W8_DEPTH.
// xrow / yrow (wave-uniform): X and Y row-major, else column-major (a lane then gathers its 8
// k-values of X with 2-byte loads, ldx apart; Y is stored column by column).  RAGGED: N is a
// multiple of 8 but not of W8_COLS (the last column block is partial).
template <int KSTEPS, bool RAGGED>
__global__ void __launch_bounds__(64 * W8_WAVES) w8a16_kernel(const f16* __restrict__ X, const int8_t* __restrict__ W,
                                                    const f16* __restrict__ scale, float* __restrict__ Y,
                                                    float* partial, unsigned* counters, int M, int N, int64_t ldx,
                                                    int64_t ldw, int64_t ldy, int splits, int ks, int total_steps,
                                                    int xrow, int yrow) {
    __shared__ __attribute__((aligned(16))) float red[W8_WAVES][16][W8_COLS];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int q = lane & 15, g = lane >> 4;
    const int cb = blockIdx.x;             // column block
    const int split = blockIdx.y;          // K split
    const int mb = blockIdx.z;             // 16-row block of X / Y
    const int n0 = cb * W8_COLS;
    const int m0 = mb * 16;
    const int s_begin = (split * W8_WAVES + w) * ks;
    const int ksteps = KSTEPS > 0 ? KSTEPS : max(0, min(ks, total_steps - s_begin));
    const int64_t k_wave = (int64_t)s_begin * W8_KSTEP;

    // A operand rows: X[m0 + q][k .. k + 8) for this lane's group; rows >= M read as 0
    const bool xrow_ok = (m0 + q) < M;
    const f16* xp = xrow ? X + (int64_t)(m0 + q) * ldx + k_wave + 8 * g : X + (k_wave + 8 * g) * ldx + (m0 + q);
    // B operand columns n0 + 8 q .. + 7; in a ragged last column block (N a multiple of 8) a lane
    // whose columns lie at or past N reads the last 8 columns instead: those MFMA columns are
    // never stored, and every load stays in flight unconditionally
    const int8_t* wp = W + (k_wave + 8 * g) * ldw + (RAGGED ? min(n0 + 8 * q, N - 8) : n0 + 8 * q);

    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const f16x8 bias = {(f16)-1152.f, (f16)-1152.f, (f16)-1152.f, (f16)-1152.f,
                        (f16)-1152.f, (f16)-1152.f, (f16)-1152.f, (f16)-1152.f};
    // Weight rows and X for W8_DEPTH steps are in flight ahead of the MFMAs (a ring in
    // registers): the stream is latency-bound otherwise, one HBM round trip per step.
    // With a runtime step count the steps run in groups of DEPTH, the ring slot a
    // compile-time constant and the count bounding them through wave-uniform branches.
    constexpr int DEPTH = KSTEPS > 0 && KSTEPS < W8_DEPTH ? KSTEPS : W8_DEPTH;
    u32x2 ring[DEPTH][8];
    uint4 xring[DEPTH];
    auto load_step = [&](int s, u32x2* rows, uint4& xa) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
            rows[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wp + ((int64_t)s * W8_KSTEP + r) * ldw));
        xa = make_uint4(0, 0, 0, 0);
        if (xrow_ok) {
            if (xrow) {
                xa = *reinterpret_cast<const uint4*>(xp + s * W8_KSTEP);
            } else {
                f16x8 xv;
#pragma unroll
                for (int j = 0; j < 8; ++j) xv[j] = xp[((int64_t)s * W8_KSTEP + j) * ldx];
                xa = __builtin_bit_cast(uint4, xv);
            }
        }
    };
    // step s from ring slot u (a compile-time constant at every call), refilling it with step s + DEPTH
    auto step = [&](int u, int s) {
        u32x2 rows[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) rows[r] = ring[u][r];
        const f16x8 a = __builtin_bit_cast(f16x8, xring[u]);
        if (s + DEPTH < ksteps) load_step(s + DEPTH, ring[u], xring[u]);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int byte = t & 3;
            uint4 bw;
            if (t < 4) {
                bw.x = w8_pair(rows[0].x, rows[1].x, byte);
                bw.y = w8_pair(rows[2].x, rows[3].x, byte);
                bw.z = w8_pair(rows[4].x, rows[5].x, byte);
                bw.w = w8_pair(rows[6].x, rows[7].x, byte);
            } else {
                bw.x = w8_pair(rows[0].y, rows[1].y, byte);
                bw.y = w8_pair(rows[2].y, rows[3].y, byte);
                bw.z = w8_pair(rows[4].y, rows[5].y, byte);
                bw.w = w8_pair(rows[6].y, rows[7].y, byte);
            }
            const f16x8 b = __builtin_bit_cast(f16x8, bw) + bias;   // exact: w = (1152 + w) - 1152
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[t], 0, 0, 0);
        }
    };
#pragma unroll
    for (int s = 0; s < DEPTH; ++s)
        if (s < ksteps) load_step(s, ring[s], xring[s]);
    if constexpr (KSTEPS > 0) {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) step(s % DEPTH, s);
    } else {
        for (int s0 = 0; s0 < ksteps; s0 += DEPTH)
#pragma unroll
            for (int u = 0; u < DEPTH; ++u)
                if (s0 + u < ksteps) step(u, s0 + u);
    }
    // acc[t] lane holds column 8q + t and rows 4g + j of this wave's partial: the 16 x 16
    // Accumulator tile t whose column c is n0 + 8c + t.  The dequant scale is applied to
    // it by the per-element callback with the scale pointer in `extras`.
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        Frag<float, 16, 16, Accumulator> f;
#pragma unroll
        for (int j = 0; j < 4; ++j) f.v[j] = acc[t][j];
        if constexpr (RAGGED)
            f = perelement(ScaleStridedBounded<8>{}, f, scale, (uint32_t)(n0 + t), (uint32_t)N);
        else
            f = perelement(ScaleStrided<8>{}, f, scale, (uint32_t)(n0 + t));
#pragma unroll
        for (int j = 0; j < 4; ++j) red[w][4 * g + j][8 * q + t] = f.v[j];
    }
    __syncthreads();

    // workgroup sum over the wavefronts: thread -> (row, 4 consecutive columns)
    const int tid = threadIdx.x;
    const int row = tid >> 5, c4 = (tid & 31) * 4;
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float a = red[0][row][c4 + i];
#pragma unroll
        for (int ww = 1; ww < W8_WAVES; ++ww) a += red[ww][row][c4 + i];
        v[i] = a;
    }
    const int grow = m0 + row;
    const bool col_ok = !RAGGED || n0 + c4 < N;   // 4 columns wholly in or out (N a multiple of 8)
    if (splits > 1) {
        // Partial block of this split, [split][mb * 16 + row][N].  The stores are agent-scope
        // atomic (coherent across the XCDs' L2 caches, written through to memory) and complete
        // (vmcnt 0) before the workgroup barrier; one thread then counts the workgroup in.
        // The last of the `splits` arrivals reads the others' blocks with agent-scope atomic
        // loads, adds all of them in split order and resets the counter for the next call.
        const int64_t rows_pad = (int64_t)gridDim.z * 16;
        float* mine = partial + ((int64_t)split * rows_pad + (int64_t)mb * 16 + row) * N + n0 + c4;
        if (col_ok) {
#pragma unroll
            for (int i = 0; i < 4; ++i) __hip_atomic_store(mine + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        __shared__ int last;
        if (tid == 0) {
            unsigned* cnt = counters + (int64_t)mb * gridDim.x + cb;
            const unsigned before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = before == (unsigned)splits - 1u;
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < splits; ++sp) {
            f32x4 pv;
            if (sp == split || !col_ok) {
                pv = v;
            } else {
                const float* other = partial + ((int64_t)sp * rows_pad + (int64_t)mb * 16 + row) * N + n0 + c4;
#pragma unroll
                for (int i = 0; i < 4; ++i) pv[i] = __hip_atomic_load(other + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            y += pv;
        }
        v = y;
    }
    if (grow < M && col_ok) {
        if (yrow) {
            float* yp = Y + (int64_t)grow * ldy + n0 + c4;
#pragma unroll
            for (int i = 0; i < 4; ++i) yp[i] = v[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) Y[grow + (int64_t)(n0 + c4 + i) * ldy] = v[i];
        }
    }
}

// W column-major (K contiguous per output column: the usual layout of a linear layer's weight,
// W^T row-major), X and Y either way (a column-major X is staged as k-lines, below; one the
// kernel cannot stage is copied row-major by the host first).  Each column's dot product streams
// contiguous memory, so a workgroup takes whole columns over all of K -- no split across
// workgroups, no exchange:
//  * a workgroup owns KM_COLS = 32 columns (two 16 x 16 MFMA tiles) of MB = 1, 2 or 4 16-row
//    blocks of X (MB by M: each dequantized W fragment feeds MB MFMAs, so W is streamed once per
//    16 MB rows); its KM_KSPLIT = 2 wavefronts take half of K each and are added through LDS at the end;
//  * a wavefront streams its 32 columns in stages of KM_SEG = 128 k: W (32 columns x 128 bytes)
//    and X (16 MB rows x 256 bytes) go straight into the wavefront's own LDS ring of 4, 3 or 2
//    stages (LDS DMA, one 128-byte run of a column per 8 lanes -- HBM serves 128-byte runs of a
//    column at ~4.8 TB/s against ~3.4 for the 64-byte runs a direct MFMA-layout load would
//    make), waited for with vmcnt: no barriers between wavefronts.  A stage's buffer is refilled
//    as soon as its fragments are in registers, before its MFMAs.  W's DMA carries the
//    nontemporal hint (W is read once; ~7 % faster);
//  * 64, 72 or 80 KB of LDS per workgroup holds the chip to two workgroups per CU, which spreads
//    a grid of a few hundred workgroups evenly (a third per CU, from a shallower ring, measured
//    slower at MB = 1);
//  * LDS rows are XOR-swizzled (16-byte slot = chunk ^ row) so the fragment reads of 16 rows hit
//    distinct banks;
//  * per 64 k, lane (n, g) = (lane % 16, lane / 16) reads 16 bytes of column n0 + 16 t + n at
//    k + 16 g for tile t: the first 8 bytes are its B operand for the k-step {16 g + j}, the last
//    8 for {16 g + 8 + j} (any assignment of k to the MFMA's k-slots works when A uses the same
//    one), and the 32 bytes of X at [m = lane % 16][k + 16 g ...] are the two A operands;
//  * int8 -> fp16 exactly: the byte (w ^ 0x80) under the high byte 0x64 is the fp16 value
//    1152 + w (v_perm_b32 against a register of 0x64 bytes), then subtract 1152;
//  * K's tail: 16-byte chunks at or past K take the out-of-range offset and read zero (in W and
//    in X); rows of X at or past M likewise.  The scale is the per-element callback.
constexpr int KM_TILES = 2;                       // 16-column MFMA tiles per wavefront
constexpr int KM_CG = 1;                          // column groups (wavefronts side by side in N)
constexpr int KM_KSPLIT = 2;                      // wavefronts side by side in K
constexpr int KM_WAVES = KM_CG * KM_KSPLIT;
constexpr int KM_WCOLS = 16 * KM_TILES;           // columns per wavefront
constexpr int KM_COLS = KM_WCOLS * KM_CG;         // columns per workgroup
constexpr int KM_SEG = 128;                       // k per stage
constexpr int KM_W_INSTR = KM_WCOLS / 8;          // W DMA instructions per stage (8 columns each)
// MB 16-row blocks of X per workgroup (1, 2 or 4): each dequantized W fragment feeds MB MFMAs, so
// W is streamed once per 16 MB rows.  The stage ring is shallower as X's share of a stage grows,
// keeping two workgroups per CU (64, 72, 80 KB of LDS).
template <int MB>
struct KmCfg {
    static_assert(MB == 1 || MB == 2 || MB == 4, "1, 2 or 4 row blocks");
    static constexpr int BUFS = MB == 1 ? 4 : (MB == 2 ? 3 : 2);          // stage ring per wavefront
    static constexpr int X_INSTR = 4 * MB;                                 // X DMA instructions (4 rows each)
    static constexpr int STAGE = KM_WCOLS * KM_SEG + 16 * MB * KM_SEG * 2;  // W, then X
    static_assert(BUFS >= 1 && BUFS <= 6, "the vmcnt waits cover up to 5 later stages");
    static_assert(BUFS * STAGE >= MB * KM_TILES * 64 * 16, "the K-range sums reuse a wavefront's ring");
};

// 8 int8 weights (two dwords, k ascending) -> the 8 fp16 values of a B operand
__device__ __forceinline__ f16x8 km_dequant(uint32_t lo, uint32_t hi) {
    const uint32_t x0 = lo ^ 0x80808080u, x1 = hi ^ 0x80808080u;
    // bytes 0-3 of the selector's source pair are the 0x64 register, 4-7 the weights
    uint4 v;
    v.x = __builtin_amdgcn_perm(x0, 0x64646464u, 0x00050004u);
    v.y = __builtin_amdgcn_perm(x0, 0x64646464u, 0x00070006u);
    v.z = __builtin_amdgcn_perm(x1, 0x64646464u, 0x00050004u);
    v.w = __builtin_amdgcn_perm(x1, 0x64646464u, 0x00070006u);
    const f16x8 bias = {(f16)-1152.f, (f16)-1152.f, (f16)-1152.f, (f16)-1152.f,
                        (f16)-1152.f, (f16)-1152.f, (f16)-1152.f, (f16)-1152.f};
    return __builtin_bit_cast(f16x8, v) + bias;   // exact: w = (1152 + w) - 1152
}

// X column-major: the stage's X is [128 k-lines][16 rows] (32-byte lines), line L stored at
// km_xline(L) -- lines 16 apart would share banks in a fragment read, the permutation moves every
// other group of 16 to the other half of the banks -- and read with ds_read_b64_tr_b16: source
// lane (jj, r4) = ((lane % 16) / 4, lane % 4) of group g points at a line and rows 4 r4 .. + 3, and
// output lane r gets the 4 lines' values of row r.
__device__ __forceinline__ int km_xline(int L) { return L ^ ((L >> 2) & 4); }
typedef short km_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) km_s16x4 km_lds_s16x4;

template <bool XROW, bool YROW, int MB>
__global__ void __launch_bounds__(64 * KM_WAVES) w8a16_kmajor_kernel(const f16* __restrict__ X,
                                                                      const int8_t* __restrict__ W,
                                                                      const f16* __restrict__ scale,
                                                                      float* __restrict__ Y, int M, int N, int K,
                                                                      int64_t ldx, int64_t ldw, int64_t ldy) {
    using Cfg = KmCfg<MB>;
    constexpr int KM_BUFS = Cfg::BUFS;
    // per wavefront: a ring of stage buffers, each W [32 columns][128 bytes] then X (4 KB per
    // 16-row block)
    __shared__ __attribute__((aligned(16))) uint8_t stage_buf[KM_WAVES][KM_BUFS][Cfg::STAGE];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cg = w % KM_CG, ks = w / KM_CG;         // column group, K range
    const int q = lane & 15, g = lane >> 4;
    // this wavefront's columns start at n0 (the last block may pass N)
    const int n0 = blockIdx.x * KM_COLS + cg * KM_WCOLS;
    const int m0 = blockIdx.y * 16 * MB;
    const int stages = (K + KM_SEG - 1) / KM_SEG;
    const int per = (stages + KM_KSPLIT - 1) / KM_KSPLIT;
    const int s_begin = min(stages, ks * per), s_end = min(stages, s_begin + per);
    const int nst = s_end - s_begin;

    // buffer resources over this workgroup's 32 columns of W and 16 rows of X
    // (a ragged last column block: the range ends at column N, so columns past it read zero)
    const v4i w_rs = make_rsrc(W + (int64_t)n0 * ldw, (uint32_t)(max(0, min(KM_WCOLS, N - n0)) * ldw));
    // (X column-major: the host keeps M a multiple of 8, so a 16-byte chunk of 8 rows is wholly
    // inside or wholly past M)
    const v4i x_rs = XROW ? make_rsrc(X + (int64_t)m0 * ldx, (uint32_t)(16 * MB * ldx * 2))
                          : make_rsrc(X + m0, (uint32_t)(K * ldx * 2));
    // W instruction i, lane l: column 8 i + l / 8, slot l % 8 holding chunk slot ^ (column % 8)
    // X row-major, instruction j, lane l: row 4 j + l / 16, slot l % 16 holding chunk slot ^ (row % 16)
    // X column-major, instruction j = 4 b + jj, lane l: row block b's LDS line 32 jj + l / 2 (holding
    // k-line km_xline of it), rows 16 b + 8 (l % 2) .. + 7
    // (either way instruction j fills the 1 KB at X + 1024 j of the stage: block b at 4 KB b)
    const int wc_lo = lane >> 3, w_slot = lane & 7;
    const int xr_lo = lane >> 4, x_slot = lane & 15;
    const int rows_ok = min(16 * MB, M - m0);
    auto issue = [&](int st, int buf) {
        const int k0 = st * KM_SEG;                   // first k of the stage
        const uint32_t lds0 = lds_addr(&stage_buf[w][buf][0]);
#pragma unroll
        for (int i = 0; i < KM_W_INSTR; ++i) {
            const int col = 8 * i + wc_lo;
            const int kb = k0 + 16 * (w_slot ^ (col & 7));
            const uint32_t off = kb < K ? (uint32_t)(col * ldw + kb) : OOB_OFS;
            dma16_stream(w_rs, off, 0, lds0 + 1024 * i);   // W is read once
        }
#pragma unroll
        for (int j = 0; j < Cfg::X_INSTR; ++j) {
            uint32_t off;
            if constexpr (XROW) {
                const int row = 4 * j + xr_lo;
                const int kx = k0 + 8 * (x_slot ^ (row & 15));
                off = (kx < K && row < rows_ok) ? (uint32_t)(row * ldx * 2 + 2 * kx) : OOB_OFS;
            } else {
                const int kx = k0 + km_xline(32 * (j & 3) + (lane >> 1));
                const int row = 16 * (j >> 2) + 8 * (lane & 1);
                off = (kx < K && row < rows_ok) ? (uint32_t)((kx * ldx + row) * 2) : OOB_OFS;
            }
            dma16(x_rs, off, 0, lds0 + KM_WCOLS * KM_SEG + 1024 * j);
        }
    };

    f32x4 acc[MB][KM_TILES];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int t = 0; t < KM_TILES; ++t) acc[b][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < KM_BUFS; ++b)
        if (b < nst) issue(s_begin + b, b);
    constexpr int PER_STAGE = KM_W_INSTR + Cfg::X_INSTR;   // DMA instructions
    for (int s = 0; s < nst; ++s) {
        // this stage's DMA done; the later stages issued (up to KM_BUFS - 1) may be in flight
        const int later = min(KM_BUFS - 1, nst - 1 - s);
        if (later >= 5)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * PER_STAGE) : "memory");
        else if (later == 4)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * PER_STAGE) : "memory");
        else if (later == 3)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * PER_STAGE) : "memory");
        else if (later == 2)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PER_STAGE) : "memory");
        else if (later == 1)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_STAGE) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const int buf = s % KM_BUFS;
        const uint8_t* wb = &stage_buf[w][buf][0];
        const uint8_t* xb = wb + KM_WCOLS * KM_SEG;
        // the stage's fragments into registers; X row q of block b, k 64 h + 16 g .. + 15 is fp16
        // chunks 8 h + 2 g and + 1, W column 16 t + q at k 64 h + 16 g is chunk 4 h + g
        f16x8 xf[MB][2][2];
        uint4 wf[2][KM_TILES];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                const uint8_t* xbb = xb + 4096 * b;
                if constexpr (XROW) {
                    const int c0 = 8 * h + 2 * g;
                    xf[b][h][0] = *reinterpret_cast<const f16x8*>(xbb + 256 * q + 16 * (c0 ^ q));
                    xf[b][h][1] = *reinterpret_cast<const f16x8*>(xbb + 256 * q + 16 * ((c0 + 1) ^ q));
                } else {
                    // lines 64 h + 16 g + 4 p + jj for the p-th group of 4 k-values
                    const int jj = (lane & 15) >> 2, r4 = lane & 3;
                    km_s16x4 v[4];
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp)
                        v[pp] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (km_lds_s16x4*)(const __attribute__((address_space(3))) uint8_t*)(
                                xbb + 32 * km_xline(64 * h + 16 * g + 4 * pp + jj) + 8 * r4));
                    xf[b][h][0] =
                        __builtin_bit_cast(f16x8, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
                    xf[b][h][1] =
                        __builtin_bit_cast(f16x8, __builtin_shufflevector(v[2], v[3], 0, 1, 2, 3, 4, 5, 6, 7));
                }
            }
#pragma unroll
            for (int t = 0; t < KM_TILES; ++t) {
                const int col = 16 * t + q;
                wf[h][t] = *reinterpret_cast<const uint4*>(wb + KM_SEG * col + 16 * ((4 * h + g) ^ (col & 7)));
            }
        }
        if (s + KM_BUFS < nst) {
            // the buffer is refilled as soon as its LDS reads have returned
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(s_begin + s + KM_BUFS, buf);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int t = 0; t < KM_TILES; ++t) {
                const f16x8 w0 = km_dequant(wf[h][t].x, wf[h][t].y), w1 = km_dequant(wf[h][t].z, wf[h][t].w);
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[b][h][0], w0, acc[b][t], 0, 0, 0);
                    acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[b][h][1], w1, acc[b][t], 0, 0, 0);
                }
            }
    }
    // the K ranges added in order through LDS: every other wavefront leaves its sums in its own
    // stage ring (its DMAs all landed at its last stage's wait, its reads all returned), and the
    // first wavefront adds them to its own and finishes
    auto red = [&](int wave, int b, int t) -> f32x4* {
        return reinterpret_cast<f32x4*>(&stage_buf[wave][0][0]) + (b * KM_TILES + t) * 64 + lane;
    };
    if (ks != 0) {
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int t = 0; t < KM_TILES; ++t) *red(w, b, t) = acc[b][t];
    }
    __syncthreads();
    if (ks != 0) return;
    // acc[b][t] lane holds column n0 + 16 t + q and rows m0 + 16 b + 4 g + j: the dequant scale by
    // the per-element callback with the scale pointer in `extras`
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int t = 0; t < KM_TILES; ++t) {
            f32x4 sum = acc[b][t];
#pragma unroll
            for (int r = 1; r < KM_KSPLIT; ++r) sum += *red(r * KM_CG + cg, b, t);
            Frag<float, 16, 16, Accumulator> f;
#pragma unroll
            for (int j = 0; j < 4; ++j) f.v[j] = sum[j];
            f = perelement(ScaleStridedBounded<1>{}, f, scale, (uint32_t)(n0 + 16 * t), (uint32_t)N);
            const int col = n0 + 16 * t + q;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = m0 + 16 * b + 4 * g + j;
                if (row < M && col < N) Y[YROW ? (int64_t)row * ldy + col : row + (int64_t)col * ldy] = f.v[j];
            }
        }
}

// A column-major X (element (m, k) at k ldx + m) copied row-major with leading dimension K,
// for the column-major-W kernel when it cannot stage X in place (M not a multiple of 8).
__global__ void w8a16_x_rows_kernel(const f16* __restrict__ X, f16* __restrict__ Xr, int64_t M, int64_t K,
                                    int64_t ldx) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= M * K) return;
    const int64_t m = e % M, k = e / M;   // consecutive threads read consecutive m of one k
    Xr[m * K + k] = X[k * ldx + m];
}

// Any layout, any shape: one thread per output element, fp32 sums.
__global__ void w8a16_generic_kernel(const f16* __restrict__ X, const int8_t* __restrict__ W,
                                     const f16* __restrict__ scale, float* __restrict__ Y, int64_t M, int64_t N,
                                     int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, uint32_t layout) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t r = idx / N, c = idx % N;
    const bool xrow = layout & 1u, wrow = layout & 2u, yrow = layout & 4u;
    float s = 0.f;
    for (int64_t k = 0; k < K; ++k) {
        const float x = (float)X[xrow ? r * ldx + k : k * ldx + r];
        const float wv = (float)W[wrow ? k * ldw + c : c * ldw + k];
        s = fmaf(x, wv, s);
    }
    Y[yrow ? r * ldy + c : c * ldy + r] = s * (float)scale[c];
}

// ---- launch planning ----------------------------------------------------------------------
enum W8Path { W8_GENERIC = 0, W8_SPLIT = 1, W8_KMAJOR = 2 };

// Arrival counters at the front of a split-K workspace: the split rule keeps splits * column
// blocks * row blocks <= 256 with splits >= 2, so at most 128 counters are ever in use.
constexpr size_t W8_COUNTER_BYTES = STREAM_WS_RESERVED;
static_assert(W8_COUNTER_BYTES >= 128 * sizeof(unsigned), "counter region");

struct W8Plan {
    W8Path path = W8_GENERIC;
    int64_t cblocks = 0, mblocks = 0, total_steps = 0, ks = 0;
    // X and Y orientation; W8_KMAJOR: X's leading dimension as the kernel reads it
    bool xrow = true, yrow = true;
    int64_t kldx = 0;
    // W8_KMAJOR with a column-major X the kernel cannot stage (M not a multiple of 8): X is first
    // copied row-major into the workspace, after the counter region
    bool x_copy = false;
    int splits = 1;
    int mb = 1;                  // W8_KMAJOR: 16-row blocks of X per workgroup
    int ksteps = 0;              // the per-wavefront step count of an unrolled instance, or 0
    // split-K workspace (W8_SPLIT with splits > 1): the arrival counters (one per column and
    // row block, zero between calls) in the first counter_bytes, then the partial blocks
    size_t counter_bytes = 0;
    size_t scratch_bytes = 0;
};

// max_scratch: the most workspace the caller can provide (the no-allocation entry's fixed array, or
// under graph capture the workspace the stream already has).
static W8Plan plan_w8a16(const void* X, const void* W, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                         uint32_t layout, size_t max_scratch) {
    W8Plan p;
    // W column-major, X and Y either way (the kernel's 32-bit buffer offsets span 32 columns of
    // W and 16 rows of X).  A column-major X of one row with unit stride is the same bytes as a
    // row-major one; otherwise a column-major X needs M a multiple of 8 (whole 16-byte chunks of
    // rows).
    bool xrow = layout & 1u;
    int64_t kldx = ldx;
    if (!xrow && M == 1 && ldx == 1) {
        xrow = true;
        kldx = K;
    }
    bool x_ok = xrow ? (kldx % 8 == 0 && kldx >= K && kldx <= (int64_t(1) << 26) && aligned(X, 16))
                     : (M % 8 == 0 && ldx % 8 == 0 && ldx >= M && K * ldx <= (int64_t(1) << 30) && aligned(X, 16));
    // otherwise a column-major X is copied row-major (leading dimension K) into the workspace
    const size_t copy_bytes = (size_t)((M * K * 2 + 255) / 256 * 256);
    const bool x_copy = !x_ok && !xrow && K <= (int64_t(1) << 26) && M * K <= (int64_t(1) << 36) &&
                        W8_COUNTER_BYTES + copy_bytes <= max_scratch;
    if ((layout & 2u) == 0 && (x_ok || x_copy) && K > 0 && K % 16 == 0 && ldw % 16 == 0 &&
        ldw >= K && ldw <= (int64_t(1) << 31) / KM_WCOLS && aligned(W, 16) && N <= 0x7fffffff && M <= 0x7fffffff &&
        (M + 15) / 16 <= 65535) {
        p.path = W8_KMAJOR;
        p.cblocks = (N + KM_COLS - 1) / KM_COLS;
        p.xrow = x_ok ? xrow : true;
        p.yrow = layout & 4u;
        p.kldx = x_ok ? kldx : K;
        // row blocks per workgroup: W streamed once per 16 mb rows (a row-major X's buffer range,
        // 32 mb rows of ldx elements, must stay below 4 GB)
        p.mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
        while (p.mb > 1 && p.xrow && 32 * p.mb * p.kldx >= (int64_t(1) << 32)) p.mb /= 2;
        p.mblocks = (M + 16 * p.mb - 1) / (16 * p.mb);
        if (!x_ok) {
            p.x_copy = true;
            p.counter_bytes = W8_COUNTER_BYTES;
            p.scratch_bytes = W8_COUNTER_BYTES + copy_bytes;
        }
        return p;
    }
    // W row-major, X and Y either way (a row-major X in 16-byte loads)
    const bool x_row = layout & 1u;
    const bool fast = (layout & 2u) && N % 8 == 0 && K > 0 && K % W8_KSTEP == 0 &&
                      K / W8_KSTEP <= 0x7fffffff && ldw % 8 == 0 && aligned(W, 8) &&
                      (x_row ? ldx % 8 == 0 && aligned(X, 16) : true) && N <= 0x7fffffff && M <= 0x7fffffff &&
                      (M + 15) / 16 <= 65535;
    if (!fast) return p;
    p.path = W8_SPLIT;
    p.xrow = x_row;
    p.yrow = layout & 4u;
    p.mblocks = (M + 15) / 16;
    p.total_steps = K / W8_KSTEP;
    p.cblocks = (N + W8_COLS - 1) / W8_COLS;
    // split K (up to 16 ways; the partial blocks cost 8 * splits bytes per output element of
    // extra traffic) while the grid still fits the 256 CUs in one round, keeping >= 4 steps per
    // wavefront: at 16 x 4096 . 4096 x 14336 the 224-workgroup grid (2 splits) streams faster
    // than the 448-workgroup one (4 splits), and 1 split (112 workgroups) is ~20 % slower
    // (and within max_scratch: under graph capture the workspace the stream already has)
    auto split_bytes = [&](int sp) {
        return W8_COUNTER_BYTES + (size_t)sp * (size_t)p.mblocks * 16 * (size_t)N * sizeof(float);
    };
    while (p.splits < 16 && p.cblocks * p.mblocks * p.splits * 2 <= 256 &&
           p.total_steps / (W8_WAVES * p.splits * 2) >= 4 && split_bytes(p.splits * 2) <= max_scratch)
        p.splits *= 2;
    p.ks = (p.total_steps + W8_WAVES * p.splits - 1) / (W8_WAVES * p.splits);
    p.ksteps = p.ks * W8_WAVES * p.splits == p.total_steps ? (int)p.ks : 0;   // unrolled instances need equal shares
    if (p.splits > 1) {
        // the counters keep a fixed place at the front of a workspace that calls of other
        // shapes reuse: every counter is zero between calls, and no partial block covers one
        p.counter_bytes = W8_COUNTER_BYTES;
        p.scratch_bytes = split_bytes(p.splits);
    }
    return p;
}

template <int KS>
static void launch_split_ks(const W8Plan& p, const void* X, const void* W, const void* scale, void* Y, float* partial,
                            unsigned* counters, int64_t M, int64_t N, int64_t ldx, int64_t ldw, int64_t ldy,
                            hipStream_t s) {
    auto kernel = N % W8_COLS == 0 ? w8a16_kernel<KS, false> : w8a16_kernel<KS, true>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)p.cblocks, (unsigned)p.splits, (unsigned)p.mblocks),
                       dim3(64 * W8_WAVES), 0, s, (const f16*)X, (const int8_t*)W, (const f16*)scale, (float*)Y, partial,
                       counters, (int)M, (int)N, ldx, ldw, ldy, p.splits, (int)p.ks, (int)p.total_steps, (int)p.xrow,
                       (int)p.yrow);
}

// Enqueues the plan's kernel on `s`.  `ws` holds p.scratch_bytes when p.splits > 1, its
// counters zero.
static int launch_w8a16(const W8Plan& p, const void* X, const void* W, const void* scale, void* Y, void* ws,
                        int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, uint32_t layout,
                        hipStream_t s) {
    if (p.path == W8_SPLIT) {
        unsigned* counters = static_cast<unsigned*>(ws);
        float* partial = ws ? reinterpret_cast<float*>(static_cast<char*>(ws) + p.counter_bytes) : nullptr;
        switch (p.ksteps) {   // the usual counts fully unrolled, any other in groups of W8_DEPTH
        case 1: launch_split_ks<1>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        case 2: launch_split_ks<2>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        case 4: launch_split_ks<4>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        case 8: launch_split_ks<8>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        case 16: launch_split_ks<16>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        case 32: launch_split_ks<32>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        default: launch_split_ks<0>(p, X, W, scale, Y, partial, counters, M, N, ldx, ldw, ldy, s); break;
        }
        LAVA_LAUNCH_CHECK("w8a16_kernel");
        return LAVA_HIP_OK;
    }
    if (p.path == W8_KMAJOR) {
        const f16* xk = (const f16*)X;
        if (p.x_copy) {
            f16* xr = reinterpret_cast<f16*>(static_cast<char*>(ws) + p.counter_bytes);
            const int64_t total = M * K;
            hipLaunchKernelGGL(w8a16_x_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                               (const f16*)X, xr, M, K, ldx);
            LAVA_LAUNCH_CHECK("w8a16_x_rows_kernel");
            xk = xr;
        }
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3((unsigned)p.cblocks, (unsigned)p.mblocks), dim3(64 * KM_WAVES), 0, s, xk,
                               (const int8_t*)W, (const f16*)scale, (float*)Y, (int)M, (int)N, (int)K, p.kldx, ldw,
                               ldy);
        };
        auto by_mb = [&](auto xr, auto yr) {
            constexpr bool XR = decltype(xr)::value, YR = decltype(yr)::value;
            if (p.mb == 4) go(w8a16_kmajor_kernel<XR, YR, 4>);
            else if (p.mb == 2) go(w8a16_kmajor_kernel<XR, YR, 2>);
            else go(w8a16_kmajor_kernel<XR, YR, 1>);
        };
        typedef std::integral_constant<bool, true> T_;
        typedef std::integral_constant<bool, false> F_;
        if (p.xrow)
            p.yrow ? by_mb(T_{}, T_{}) : by_mb(T_{}, F_{});
        else
            p.yrow ? by_mb(F_{}, T_{}) : by_mb(F_{}, F_{});
        LAVA_LAUNCH_CHECK(p.mb == 1 ? "w8a16_kmajor_kernel" : (p.mb == 2 ? "w8a16_kmajor_kernel<mb2>"
                                                                          : "w8a16_kmajor_kernel<mb4>"));
        return LAVA_HIP_OK;
    }
    // any layout, any shape
    const int64_t total = M * N;
    hipLaunchKernelGGL(w8a16_generic_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, (const f16*)X,
                       (const int8_t*)W, (const f16*)scale, (float*)Y, M, N, K, ldx, ldw, ldy, layout);
    LAVA_LAUNCH_CHECK("w8a16_generic_kernel");
    return LAVA_HIP_OK;
}

static int check_w8a16_args(const void* X, const void* W, const void* scale, const void* Y, int64_t M, int64_t N,
                            int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, uint32_t layout, const char* name) {
    LAVA_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative extent (M=%lld N=%lld K=%lld)", name, (long long)M,
             (long long)N, (long long)K);
    LAVA_ARG(layout <= 7u, "%s: layout %u has bits beyond X/W/Y row-major", name, layout);
    if (M == 0 || N == 0) return LAVA_HIP_OK;
    LAVA_ARG(Y != nullptr && scale != nullptr, "%s: null Y or scale", name);
    LAVA_ARG(K == 0 || (X != nullptr && W != nullptr), "%s: null X or W", name);
    const bool xrow = layout & 1u, wrow = layout & 2u, yrow = layout & 4u;
    LAVA_ARG(ldx >= (xrow ? (K > 0 ? K : 1) : M), "%s: ldx = %lld too small", name, (long long)ldx);
    LAVA_ARG(ldw >= (wrow ? N : (K > 0 ? K : 1)), "%s: ldw = %lld too small", name, (long long)ldw);
    LAVA_ARG(ldy >= (yrow ? N : M), "%s: ldy = %lld too small", name, (long long)ldy);
    LAVA_ARG(aligned(X, 2) && aligned(scale, 2) && aligned(Y, 4), "%s: misaligned X, scale or Y", name);
    LAVA_REQUIRE((M * N + 255) / 256 <= 0x7fffffff && M * (N / 4) / 256 < 0x7fffffff, LAVA_HIP_ERR_UNSUPPORTED,
                 "%s: problem too large", name);
    return LAVA_HIP_OK;
}

// ---- the per-stream workspace (W8A16 and the small-product GEMM's split-K) -------------------
// One buffer per (device, stream), owned by the library.  The lock is held from the
// workspace lookup through the launch, so calls from several threads on one stream use the
// workspace one after another (stream order).  A buffer that grows is retired, not freed --
// work already enqueued may still use it -- and every buffer of a stream is freed by
// lava_hip_stream_destroy (after the stream drains) or lava_hip_release_workspaces (after the
// device drains).  A stream that is capturing a graph never allocates (hipMalloc is not
// capturable): its calls plan within the buffer it has (stream_workspace_cap), and that buffer
// is marked as held by a graph, which may replay it after the stream is gone, so it is moved
// to g_ws_kept instead of being freed.
struct W8Workspace {
    void* buf = nullptr;
    size_t bytes = 0;
    bool captured = false;          // a graph captured on the stream holds buf
    std::vector<void*> retired;
};
static std::mutex g_ws_mutex;
static std::map<std::pair<int, void*>, W8Workspace> g_ws;
static std::vector<void*> g_ws_kept;    // buffers graphs may hold: kept until the process ends

// Whether `stream` is capturing a graph; a failed query counts as capturing (the caller then
// does not allocate), and its error is taken off HIP's last-error slot so that the next launch
// check does not report it.
static bool stream_capturing(void* stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(as_stream(stream), &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;
    }
    return st != hipStreamCaptureStatusNone;
}

size_t stream_workspace_cap(void* stream) {
    if (!stream_capturing(stream)) return SIZE_MAX;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    auto it = g_ws.find({dev, stream});
    return it == g_ws.end() ? 0 : it->second.bytes;
}

int with_stream_workspace(size_t bytes, void* stream, const std::function<int(void*)>& launch) {
    int dev = 0;
    LAVA_HIP_TRY(hipGetDevice(&dev));
    const bool capturing = stream_capturing(stream);
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    W8Workspace& ws = g_ws[{dev, stream}];
    bytes = bytes < STREAM_WS_RESERVED ? STREAM_WS_RESERVED : bytes;
    if (ws.bytes < bytes) {
        LAVA_REQUIRE(!capturing, LAVA_HIP_ERR_UNSUPPORTED,
                     "the stream is capturing a graph and its workspace (%zu bytes) is smaller than this call needs "
                     "(%zu bytes): make one call of this shape outside capture first", ws.bytes, bytes);
        void* buf = nullptr;
        LAVA_HIP_TRY(hipMalloc(&buf, bytes));
        // the W8A16 arrival counters start at zero (every call leaves them at zero)
        const int rc = lava_hip_fill_bytes(buf, 0, STREAM_WS_RESERVED, stream);
        if (rc != LAVA_HIP_OK) {
            (void)hipFree(buf);
            return rc;
        }
        if (ws.buf) (ws.captured ? g_ws_kept : ws.retired).push_back(ws.buf);
        ws.buf = buf;
        ws.bytes = bytes;
        ws.captured = false;
    }
    if (capturing) ws.captured = true;
    return launch(ws.buf);
}

// Frees (or, if a graph may hold it, keeps) every buffer of one workspace entry, on its device.
static void release_entry(int dev, W8Workspace& ws) {
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(dev);
    for (void* b : ws.retired) (void)hipFree(b);
    if (ws.buf) {
        if (ws.captured)
            g_ws_kept.push_back(ws.buf);
        else
            (void)hipFree(ws.buf);
    }
    (void)hipSetDevice(cur);
}

void w8a16_release_stream(void* stream) {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    for (auto it = g_ws.begin(); it != g_ws.end();) {
        if (it->first.second != stream) {
            ++it;
            continue;
        }
        release_entry(it->first.first, it->second);
        it = g_ws.erase(it);
    }
}

// ---- the no-allocation entry's scratch --------------------------------------------------------
// lava_hip_gemm_w8a16_noalloc keeps its split-K workspace (arrival counters, then partial
// blocks) in this fixed device array, one copy per GPU, reached through the address
// hipGetSymbolAddress returns for it on that GPU (the array's name is only a host-side
// stand-in).  The split rule keeps a grid at <= 256 workgroups, each writing one 16 x 128 fp32
// block, so no plan needs more than the counters plus 2 MiB.  The counters are cleared by a
// fill kernel on the first call per device; every call leaves them at zero, and every block a
// reduction reads is written by the same call first.
static_assert(LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES >= W8_COUNTER_BYTES + 256 * 16 * W8_COLS * sizeof(float),
              "the no-allocation scratch must hold the largest split-K plan");
static __device__ __attribute__((used)) __align__(256) float scratch[LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES / sizeof(float)];
constexpr int W8_MAX_DEVICES = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[W8_MAX_DEVICES];

// The device address of `scratch` on the current device, looked up (and its counters cleared,
// on `stream`) once per device.
static int scratch_for_device(void** out, void* stream) {
    int dev = 0;
    LAVA_HIP_TRY(hipGetDevice(&dev));
    LAVA_REQUIRE(dev >= 0 && dev < W8_MAX_DEVICES, LAVA_HIP_ERR_UNSUPPORTED,
                 "gemm_w8a16_noalloc: device %d beyond the %d this library tracks", dev, W8_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        LAVA_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        LAVA_REQUIRE(ptr != nullptr, LAVA_HIP_ERR_HIP, "gemm_w8a16_noalloc: no device address for the scratch array");
        const int rc = lava_hip_fill_bytes(ptr, 0, W8_COUNTER_BYTES, stream);
        if (rc != LAVA_HIP_OK) return rc;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return LAVA_HIP_OK;
}

}  // namespace lava

using namespace lava;

extern "C" int lava_hip_release_workspaces(void) {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    int cur = 0;
    LAVA_HIP_TRY(hipGetDevice(&cur));
    std::set<int> devs;
    for (auto& e : g_ws) devs.insert(e.first.first);
    for (int d : devs) {   // the buffers' last users may still be queued on any stream of the device
        LAVA_HIP_TRY(hipSetDevice(d));
        const hipError_t e = hipDeviceSynchronize();
        (void)hipSetDevice(cur);
        LAVA_HIP_TRY(e);
    }
    for (auto& e : g_ws) release_entry(e.first.first, e.second);
    g_ws.clear();
    return LAVA_HIP_OK;
}

extern "C" int lava_hip_gemm_w8a16(const void* X, const void* W, const void* scale, void* Y, int64_t M, int64_t N,
                                   int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, uint32_t layout, void* stream) {
    int rc = check_w8a16_args(X, W, scale, Y, M, N, K, ldx, ldw, ldy, layout, "gemm_w8a16");
    if (rc != LAVA_HIP_OK || M == 0 || N == 0) return rc;
    rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    // planned within the workspace the stream has when it is capturing a graph
    const W8Plan p = plan_w8a16(X, W, M, N, K, ldx, ldw, layout, stream_workspace_cap(stream));
    hipStream_t s = as_stream(stream);
    if (p.scratch_bytes == 0) return launch_w8a16(p, X, W, scale, Y, nullptr, M, N, K, ldx, ldw, ldy, layout, s);
    return with_stream_workspace(p.scratch_bytes, stream, [&](void* ws) {
        return launch_w8a16(p, X, W, scale, Y, ws, M, N, K, ldx, ldw, ldy, layout, s);
    });
}

extern "C" int lava_hip_gemm_w8a16_noalloc(const void* X, const void* W, const void* scale, void* Y, int64_t M,
                                           int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy,
                                           uint32_t layout, void* stream) {
    int rc = check_w8a16_args(X, W, scale, Y, M, N, K, ldx, ldw, ldy, layout, "gemm_w8a16_noalloc");
    if (rc != LAVA_HIP_OK || M == 0 || N == 0) return rc;
    const W8Plan p = plan_w8a16(X, W, M, N, K, ldx, ldw, layout, LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES);
    LAVA_ARG(p.scratch_bytes <= LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES,
             "gemm_w8a16_noalloc: this shape needs %zu bytes of split-K scratch; the no-allocation entry holds at most "
             "%zu (M = %lld, N = %lld, K = %lld)", p.scratch_bytes, (size_t)LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES,
             (long long)M, (long long)N, (long long)K);
    rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;
    void* ws = nullptr;
    if (p.scratch_bytes > 0) {
        rc = scratch_for_device(&ws, stream);
        if (rc != LAVA_HIP_OK) return rc;
    }
    return launch_w8a16(p, X, W, scale, Y, ws, M, N, K, ldx, ldw, ldy, layout, as_stream(stream));
}
