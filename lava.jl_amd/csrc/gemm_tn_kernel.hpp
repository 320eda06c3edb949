// gemm_tn_kernel.hpp -- the compute-bound GEMM kernel (gemm_tn16_kernel), C row-major,
// every operand layout.
//
// This is the staged cooperative-matrix GEMM (src/device/coopmat_intrinsics.jl:
// 104-148 stages A and B through workgroup memory and reads A RowMajor and B
// ColumnMajor from the same block; test/glsl/coopmat2_gemm_regs.comp:46-84 is the
// same loop at workgroup scope) laid out for CDNA4:
//
//  * one 256 x 256 tile of C per workgroup of 4 wavefronts (one per SIMD), each
//    wavefront owning a 128 x 128 sub-tile = 8 x 8 MFMA 16x16 accumulators (256 fp32
//    registers per lane, all in AGPRs);
//  * K advances 128 bytes at a time (64 bf16/fp16 or 128 int8): A and B slices of
//    32 KB each, double-buffered in LDS (2 x 64 KB);
//  * global -> LDS with buffer_load_dwordx4 ... lds: each lane moves 16 bytes
//    straight into LDS, no register staging, addressed by a buffer resource plus a
//    32-bit lane offset (the wave-uniform parts in soffset); one wavefront
//    instruction fills 1 KB of LDS, lane l the 16-byte slot l;
//  * each operand is staged in one of two forms, chosen by its layout (TnSide):
//    K-contiguous (A row-major, B column-major), 256 rows x 128 bytes of K, or
//    M/N-contiguous (A column-major, B row-major; 16-bit types), 64 rows of K x 512
//    bytes; 16-byte chunks XOR-swizzled per row, chosen by which global chunk each lane
//    fetches, so that the fragment reads are bank-conflict-free;
//  * a fragment is 16 bytes per lane (one ds_read_b128, or two transposing
//    ds_read_b64_tr_b16 for an M/N-contiguous operand); per stage two k-steps of 64
//    bytes, 64 MFMAs each, one barrier in the middle of the stage (gemm_tn16_kernel);
//  * the MFMA's A operand is the B slice and its B operand the A slice, so each
//    lane's accumulator holds runs of 4 consecutive columns of one row of C; the
//    epilogue stages them through LDS and stores whole 512-byte row runs;
//  * workgroups are renumbered XCD by XCD (xcd_tile) so that the tiles one XCD
//    runs together share rows of A and columns of B in its L2;
//  * C is written with nontemporal stores (8192^3 bf16: ~4 % faster than plain stores;
//    the HBM fetch of A and B is unchanged, so the gain is on the write side);
//  * ragged extents (the RAGGED instances; Lava's TENSOR_CLAMP_CONSTANT layout with
//    the default zero, src/vocabulary/tensor.jl:44-51): a lane whose row or chunk lies
//    past M, N or K gets a lane offset beyond the buffer resource's range, so its
//    load reads zero instead of memory; the store and the epilogue's operand loads
//    are bounds-checked.  A K-contiguous operand needs K a multiple of the 16-byte
//    chunk (8 f16/bf16, 16 int8), an M/N-contiguous one M (N) a multiple of 8, so
//    that a chunk is wholly in or out.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gemm_common.hpp"
#include "gemm_kernels.hpp"
#include "lds_dma.hpp"
#include "lava_hip_internal.hpp"

namespace lava {

constexpr int TN_TILE = 256;    // rows of A / columns of B per workgroup
constexpr int TN_KB = 128;      // bytes of K per stage
constexpr int TN_SLICE = TN_TILE * TN_KB;  // 32 KB

typedef short tn_s16x4 __attribute__((ext_vector_type(4)));
typedef int tn_v2i __attribute__((ext_vector_type(2)));
typedef short tn_s16x8 __attribute__((ext_vector_type(8)));

// The M/N-contiguous swizzle F(r % 4) = {0, 6, 10, 12}, as nibbles.
__device__ __forceinline__ int tn_mn_swz(int r4) { return (0xCA60 >> (4 * r4)) & 0xF; }

// One operand's staging: DMA offsets and validity, and its fragment reads.  TILE: rows (m or n)
// of the operand per workgroup tile -- 256 for the tile kernel; the K-contiguous form also serves
// the 128 x 128 mid-size kernel (gemm_mid.hip).
template <typename T, bool KC, int TILE = TN_TILE>
struct TnSide;

// K-contiguous: the slice is TILE rows (m or n) x 128 bytes of K.  Row r's logical
// 16-byte chunk c is stored at slot c ^ (r % 8): a 16x16 fragment read (16 consecutive
// rows, one chunk per 16 lanes) then hits every bank once.  (With an extra ^ (r / 8 % 2),
// the swizzle a 32-row read needs, the 16-row read costs ~4 conflict cycles; measured with
// SQ_LDS_BANK_CONFLICT.)
template <typename T, int TILE>
struct TnSide<T, true, TILE> {
    static constexpr int WROWS = TILE / 4;   // rows one wavefront's DMAs fill
    static constexpr int HALF = TILE / 2;    // rows one wavefront's fragments read
    v4i rs;
    uint32_t off;      // the lane's row and chunk within an instruction's 8 rows
    uint32_t step;     // soffset per instruction: 8 rows
    int lim;           // instruction i's rows are inside iff 8 i < lim
    int kend;          // last byte (+1) of the lane's chunk
    int rd16, sl16[2];   // fragment reads: row offset, chunk slot per k-step

    // rows_in: rows of this tile inside the matrix; w: the wavefront; wx: its 128-row half.
    __device__ __forceinline__ void init(const T* X, int64_t ld_b, int tile, int rows_in, int64_t, int, int w, int wx,
                                         int lane) {
        rs = make_rsrc(reinterpret_cast<const char*>(X) + (int64_t)tile * TILE * ld_b,
                       (uint32_t)(rows_in * ld_b));
        // DMA: an instruction covers 8 rows; lane l row l / 8, slot l % 8, which holds chunk slot ^ row % 8
        const int lr = lane >> 3;
        const int c = (lane & 7) ^ lr;
        off = (uint32_t)((WROWS * w + lr) * ld_b + 16 * c);
        step = (uint32_t)(8 * ld_b);
        lim = rows_in - WROWS * w - lr;
        kend = 16 * c + 16;
        // fragments: row 16 t + lane % 16 of the half, chunk 4 u + lane / 16
        rd16 = (wx * HALF + (lane & 15)) * TN_KB;
#pragma unroll
        for (int u = 0; u < 2; ++u) sl16[u] = ((4 * u + (lane >> 4)) ^ (lane & 7)) * 16;
    }
    __device__ __forceinline__ bool valid(int i, uint32_t kofs, int kb) const {
        return 8 * i < lim && (int)kofs + kend <= kb;
    }
    __device__ __forceinline__ uint32_t voff(int) const { return off; }
    __device__ __forceinline__ uint32_t soff(int i, uint32_t kofs) const { return i * step + kofs; }
    // fragment t (rows 16 t of the half) of k-step u (64 bytes of K)
    __device__ __forceinline__ uint4 read16(const uint8_t* slice, int u, int t) const {
        return *reinterpret_cast<const uint4*>(slice + rd16 + t * 16 * TN_KB + sl16[u]);
    }
};

// M/N-contiguous (16-bit): the slice is 64 rows of K x 512 bytes (256 m or n).  Row r's
// logical 16-byte chunk c is stored at slot c ^ F(r % 4) ^ 8 (r / 8 % 4), F = {0, 6, 10, 12}:
// a 16x16 fragment is two transposing reads (ds_read_b64_tr_b16: in a 16-lane group,
// output lane i value j is the 16-bit word at source lane 4 j + i / 4's address
// + 2 (i % 4)), whose 16 k rows (4 groups of 4, 8 apart) x 32 bytes that swizzle spreads
// over all banks (without the r / 8 term, ~2 conflict cycles per read; SQ_LDS_BANK_CONFLICT).
template <typename T>
struct TnSide<T, false, TN_TILE> {
    static_assert(sizeof(T) == 2, "M/N-contiguous staging reads 16-bit elements transposed");
    v4i rs;
    uint32_t off[4];   // per instruction variant (i % 2, i / 4): the row's swizzle depends on them
    uint32_t step;     // soffset per instruction: 2 rows of K
    uint32_t ld;       // bytes per row of K
    int klim;          // instruction i's row is inside iff k0 + 2 i < klim
    bool cin[4];       // the lane's chunk lies inside M (N), per variant
    int mr16;          // fragment reads: the lane's row and byte offset
    int c16[8];        // fragment reads: the stored chunk of column block t, times 16

    // mn_total: M (N); K: the depth in elements; w: the wavefront; wx: its 128-column half.
    __device__ __forceinline__ void init(const T* X, int64_t ld_b, int tile, int, int64_t mn_total, int K, int w,
                                         int wx, int lane) {
        const int64_t col0 = (int64_t)tile * TN_TILE;
        rs = make_rsrc(reinterpret_cast<const char*>(X) + col0 * (int64_t)sizeof(T),
                       (uint32_t)((int64_t)K * ld_b - col0 * (int64_t)sizeof(T)));
        // DMA: instruction i covers rows 16 w + 2 i + h (h = lane / 32), slot lane % 32; that
        // row's r % 4 is 2 (i % 2) + h and r / 8 % 4 is (2 w + i / 4) % 4
        const int h = lane >> 5, p = lane & 31;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int c = p ^ tn_mn_swz((2 * (v & 1) + h) & 3) ^ (((2 * w + (v >> 1)) & 3) << 3);
            off[v] = (uint32_t)((16 * w + h) * ld_b + 16 * c);
            cin[v] = col0 + 8 * c < mn_total;
        }
        step = (uint32_t)(2 * ld_b);
        ld = (uint32_t)ld_b;
        klim = K - 16 * w - h;
        // fragments: source lane ss of 16-lane group g points at k row 8 g + 4 r + ss / 4
        // (+ 32 u), columns 16 t + 4 (ss % 4) of the half; that row's swizzle is
        // F(ss / 4) ^ 8 g for every u, t and r
        const int ss = lane & 15, g = lane >> 4;
        const int f = tn_mn_swz(ss >> 2) ^ (g << 3);
        mr16 = (8 * g + (ss >> 2)) * 512 + 8 * (ss & 1);
#pragma unroll
        for (int t = 0; t < 8; ++t) c16[t] = ((16 * wx + 2 * t + ((ss & 3) >> 1)) ^ f) * 16;
    }
    __device__ __forceinline__ static int variant(int i) { return (i & 1) | ((i >> 2) << 1); }
    __device__ __forceinline__ bool valid(int i, uint32_t kofs, int) const {
        return (int)(kofs / sizeof(T)) + 2 * i < klim && cin[variant(i)];
    }
    __device__ __forceinline__ uint32_t voff(int i) const { return off[variant(i)]; }
    __device__ __forceinline__ uint32_t soff(int i, uint32_t kofs) const {
        return (kofs / (uint32_t)sizeof(T)) * ld + i * step;
    }
    // fragment t (columns 16 t of the half) of k-step u (32 rows of K): two transposing
    // reads, k rows 8 g + [0, 4) and 8 g + [4, 8) of the k-step
    __device__ __forceinline__ uint4 read16(const uint8_t* slice, int u, int t) const {
        const uint8_t* b = slice + u * 32 * 512 + mr16 + c16[t];
        const tn_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) tn_s16x4*)(const __attribute__((address_space(3))) uint8_t*)b);
        const tn_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) tn_s16x4*)(const __attribute__((address_space(3))) uint8_t*)(b + 4 * 512));
        return __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
};

// M/N-contiguous (16-bit) at 128 columns per tile (the mid-size kernel): the slice is 64 rows of K x
// 256 bytes, one bank window per row.  Row r's logical 16-byte chunk c is stored at slot c ^ S(r),
// S(r) = 2 (r % 4) + 8 ((r / 8 + r / 16) % 2).  A fragment's transposing read touches 16 k rows (the
// 4-row groups 8 g + [0, 4) of the four 16-lane groups g) x 2 adjacent chunks; whether the hardware
// serves it as lanes 0-31 and 32-63 (rows 8 g, g = 0, 1 or 2, 3: row bits 0, 1 and 3 vary) or as lane
// groups {0, 2} and {1, 3} (bits 0, 1 and 4), S gives the 8 rows of a pass distinct chunk pairs
// (bits 1-3 of the slot), so the 16 chunk reads of a pass cover a 256-byte window once.
template <typename T>
struct TnSide<T, false, 128> {
    static_assert(sizeof(T) == 2, "M/N-contiguous staging reads 16-bit elements transposed");
    v4i rs;
    uint32_t off[2];   // per instruction variant i / 2: the row's swizzle depends on it
    uint32_t step;     // soffset per instruction: 4 rows of K
    uint32_t ld;       // bytes per row of K
    int klim;          // instruction i's row is inside iff k0 + 4 i < klim
    bool cin[2];       // the lane's chunk lies inside M (N), per variant
    int mr16;          // fragment reads: the lane's row and byte offset
    int c16[4];        // fragment reads: the stored chunk of column block t, times 16

    __device__ __forceinline__ static int swz(int r) { return 2 * (r & 3) + 8 * (((r >> 3) ^ (r >> 4)) & 1); }

    // mn_total: M (N); K: the depth in elements; w: the wavefront; wx: its 64-column half.
    __device__ __forceinline__ void init(const T* X, int64_t ld_b, int tile, int, int64_t mn_total, int K, int w,
                                         int wx, int lane) {
        const int64_t col0 = (int64_t)tile * 128;
        rs = make_rsrc(reinterpret_cast<const char*>(X) + col0 * (int64_t)sizeof(T),
                       (uint32_t)((int64_t)K * ld_b - col0 * (int64_t)sizeof(T)));
        // DMA: instruction i covers k rows 16 w + 4 i + lane / 16, slot lane % 16; that row's
        // swizzle is S(16 w + 4 i + lane / 16): bits 0, 1 from lane / 16, bit 3 from i / 2, bit 4 from w
        const int rr = lane >> 4, p = lane & 15;
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int c = p ^ swz(16 * w + 4 * (2 * v) + rr);
            off[v] = (uint32_t)((16 * w + rr) * ld_b + 16 * c);
            cin[v] = col0 + 8 * c < mn_total;
        }
        step = (uint32_t)(4 * ld_b);
        ld = (uint32_t)ld_b;
        klim = K - 16 * w - rr;
        // fragments: source lane ss of 16-lane group g points at k row 8 g + 4 r + ss / 4 (+ 32 u),
        // columns 16 t + 4 (ss % 4) of the half; that row's swizzle is S(8 g + ss / 4) for every
        // u, t and r (bit 2 and bit 5 do not enter S)
        const int ss = lane & 15, g = lane >> 4;
        const int f = swz(8 * g + (ss >> 2));
        mr16 = (8 * g + (ss >> 2)) * 256 + 8 * (ss & 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) c16[t] = ((8 * wx + 2 * t + ((ss & 3) >> 1)) ^ f) * 16;
    }
    __device__ __forceinline__ bool valid(int i, uint32_t kofs, int) const {
        return (int)(kofs / sizeof(T)) + 4 * i < klim && cin[i >> 1];
    }
    __device__ __forceinline__ uint32_t voff(int i) const { return off[i >> 1]; }
    __device__ __forceinline__ uint32_t soff(int i, uint32_t kofs) const {
        return (kofs / (uint32_t)sizeof(T)) * ld + i * step;
    }
    // fragment t (columns 16 t of the half) of k-step u (32 rows of K): two transposing reads, k rows
    // 8 g + [0, 4) and 8 g + [4, 8) of the k-step
    __device__ __forceinline__ uint4 read16(const uint8_t* slice, int u, int t) const {
        const uint8_t* b = slice + u * 32 * 256 + mr16 + c16[t];
        const tn_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) tn_s16x4*)(const __attribute__((address_space(3))) uint8_t*)b);
        const tn_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) tn_s16x4*)(const __attribute__((address_space(3))) uint8_t*)(b + 4 * 256));
        return __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
};

// M/N-contiguous int8: the slice is 128 rows of K x 256 bytes (256 m or n).  Row r's logical
// 16-byte chunk c is stored at slot c ^ F8(r), F8(r) = (r % 8) | 8 (r / 16 % 2).  A fragment is
// two transposing reads (ds_read_b64_tr_b8: in a 16-lane group, output lane i byte j is the
// byte at source lane 2 j + i / 8's address + i % 8; measured on the box).  Source lane s of
// 16-lane group g points at k row 64 u + 16 g + 8 h + s / 2 of k-step u (h = 0, 1 for the two
// reads), byte 8 (s % 2) of the block's chunk, so output lane i receives the k-values
// 64 u + 16 g + 8 h + [0, 8) of column 16 t + i: together the 16 k-slots a K-contiguous
// fragment gives lane group g (bytes 16 g .. 16 g + 15 of the k-step), so the two forms mix.
// F8 puts the 8 rows one group reads, and the two groups of a 32-lane half, on distinct banks.
template <>
struct TnSide<int8_t, false, TN_TILE> {
    v4i rs;
    uint32_t off[4];   // per instruction variant (i % 2, i / 4): the row's swizzle depends on them
    uint32_t step;     // soffset per instruction: 4 rows of K
    uint32_t ld;       // bytes per row of K
    int klim;          // instruction i's row is inside iff k0 + 4 i < klim
    bool cin[4];       // the lane's chunk lies inside M (N), per variant
    int rd;            // fragment reads: the lane's k row and byte offset
    int c16[8];        // fragment reads: the stored chunk of column block t, times 16

    // mn_total: M (N); K: the depth in elements; w: the wavefront; wx: its 128-column half.
    __device__ __forceinline__ void init(const int8_t* X, int64_t ld_b, int tile, int, int64_t mn_total, int K, int w,
                                         int wx, int lane) {
        const int64_t col0 = (int64_t)tile * TN_TILE;
        rs = make_rsrc(reinterpret_cast<const char*>(X) + col0, (uint32_t)((int64_t)K * ld_b - col0));
        // DMA: instruction i covers rows 32 w + 4 i + lane / 16, slot lane % 16; that row's
        // r % 8 is 4 (i % 2) + lane / 16 and r / 16 % 2 is i / 4
        const int rr = lane >> 4, p = lane & 15;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int c = p ^ ((4 * (v & 1) + rr) | ((v >> 1) << 3));
            off[v] = (uint32_t)((32 * w + rr) * ld_b + 16 * c);
            cin[v] = col0 + 16 * c < mn_total;
        }
        step = (uint32_t)(4 * ld_b);
        ld = (uint32_t)ld_b;
        klim = K - 32 * w - rr;
        // fragments: every row a lane reads has F8 = (s / 2) | 8 (g % 2)
        const int s = lane & 15, g = lane >> 4;
        const int f = (s >> 1) | ((g & 1) << 3);
        rd = (16 * g + (s >> 1)) * 256 + 8 * (s & 1);
#pragma unroll
        for (int t = 0; t < 8; ++t) c16[t] = ((8 * wx + t) ^ f) * 16;
    }
    __device__ __forceinline__ static int variant(int i) { return (i & 1) | ((i >> 2) << 1); }
    __device__ __forceinline__ bool valid(int i, uint32_t kofs, int) const {
        return (int)kofs + 4 * i < klim && cin[variant(i)];
    }
    __device__ __forceinline__ uint32_t voff(int i) const { return off[variant(i)]; }
    __device__ __forceinline__ uint32_t soff(int i, uint32_t kofs) const { return kofs * ld + i * step; }
    // fragment t (columns 16 t of the half) of k-step u (64 rows of K): two transposing reads,
    // k rows 16 g + [0, 8) and 16 g + [8, 16) of the k-step
    __device__ __forceinline__ uint4 read16(const uint8_t* slice, int u, int t) const {
        const uint8_t* b = slice + u * 64 * 256 + rd + c16[t];
        const tn_v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) tn_v2i*)(const __attribute__((address_space(3))) uint8_t*)b);
        const tn_v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) tn_v2i*)(const __attribute__((address_space(3))) uint8_t*)(b + 8 * 256));
        return make_uint4((uint32_t)lo.x, (uint32_t)lo.y, (uint32_t)hi.x, (uint32_t)hi.y);
    }
};

// M/N-contiguous int8 at 128 columns per tile (the mid-size kernel): the slice is 128 rows of K x 128
// bytes, two rows per 256-byte bank window.  Row r's logical chunk c is stored at slot c ^ F(r),
// F(r) = (r / 2 % 4) | 4 ((r / 16 + r / 32) % 2).  The transposing reads are the 256-column form's
// (source lane s of 16-lane group g at k row 64 u + 16 g + 8 h + s / 2, byte 8 (s % 2) of the
// fragment's chunk); a 32-lane pass reads 16 rows x one chunk, and F gives the rows of each parity
// distinct slots whether the pass is groups {0, 1} (row bit 4 varies) or {0, 2} / {1, 3} (bit 5), so
// the pass's 16 chunk reads (row parity x slot) cover the 256-byte window once.
template <>
struct TnSide<int8_t, false, 128> {
    v4i rs;
    uint32_t off[2];   // per instruction variant i / 2: the row's swizzle depends on it
    uint32_t step;     // soffset per instruction: 8 rows of K
    uint32_t ld;       // bytes per row of K
    int klim;          // instruction i's row is inside iff k0 + 8 i < klim
    bool cin[2];       // the lane's chunk lies inside M (N), per variant
    int rd;            // fragment reads: the lane's k row and byte offset
    int c16[4];        // fragment reads: the stored chunk of column block t, times 16

    __device__ __forceinline__ static int swz(int r) { return ((r >> 1) & 3) | ((((r >> 4) ^ (r >> 5)) & 1) << 2); }

    // mn_total: M (N); K: the depth in elements; w: the wavefront; wx: its 64-column half.
    __device__ __forceinline__ void init(const int8_t* X, int64_t ld_b, int tile, int, int64_t mn_total, int K, int w,
                                         int wx, int lane) {
        const int64_t col0 = (int64_t)tile * 128;
        rs = make_rsrc(reinterpret_cast<const char*>(X) + col0, (uint32_t)((int64_t)K * ld_b - col0));
        // DMA: instruction i covers k rows 32 w + 8 i + lane / 8, slot lane % 8; that row's swizzle
        // is F(32 w + 8 i + lane / 8): bits 1, 2 from lane / 8, bit 4 from i / 2, bit 5 from w
        const int rr = lane >> 3, p = lane & 7;
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int c = p ^ swz(32 * w + 16 * v + rr);
            off[v] = (uint32_t)((32 * w + rr) * ld_b + 16 * c);
            cin[v] = col0 + 16 * c < mn_total;
        }
        step = (uint32_t)(8 * ld_b);
        ld = (uint32_t)ld_b;
        klim = K - 32 * w - rr;
        // fragments: every row a lane reads (16 g + 8 h + s / 2 + 64 u) has F = (s / 4) | 4 (g % 2 ^ g / 2)
        const int s = lane & 15, g = lane >> 4;
        const int f = swz(16 * g + (s >> 1));
        rd = (16 * g + (s >> 1)) * 128 + 8 * (s & 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) c16[t] = ((4 * wx + t) ^ f) * 16;
    }
    __device__ __forceinline__ bool valid(int i, uint32_t kofs, int) const {
        return (int)kofs + 8 * i < klim && cin[i >> 1];
    }
    __device__ __forceinline__ uint32_t voff(int i) const { return off[i >> 1]; }
    __device__ __forceinline__ uint32_t soff(int i, uint32_t kofs) const { return kofs * ld + i * step; }
    // fragment t (columns 16 t of the half) of k-step u (64 rows of K): two transposing reads,
    // k rows 16 g + [0, 8) and 16 g + [8, 16) of the k-step
    __device__ __forceinline__ uint4 read16(const uint8_t* slice, int u, int t) const {
        const uint8_t* b = slice + u * 64 * 128 + rd + c16[t];
        const tn_v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) tn_v2i*)(const __attribute__((address_space(3))) uint8_t*)b);
        const tn_v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) tn_v2i*)(const __attribute__((address_space(3))) uint8_t*)(b + 8 * 128));
        return make_uint4((uint32_t)lo.x, (uint32_t)lo.y, (uint32_t)hi.x, (uint32_t)hi.y);
    }
};

// The tile kernel.  AK / BK: A / B K-contiguous (row-major A, column-major B) or
// M/N-contiguous (transposing LDS reads, 16- or 8-bit).  16x16 MFMAs (16x16x32 for 16-bit
// types, 16x16x64 for int8), 8 x 8 accumulators of 16 x 16 per wavefront: at the chip's
// power limit the 16x16 shape sustains ~11 % more than 32x32 (it moves ~20 % fewer
// register-file bytes per flop), and its fragments (16 rows x 64 bytes of K per k-step)
// let the whole stage be read by the middle of the k-tile, so that the barrier sits there
// and each DMA gets a full k-tile to land.
//
// U8 (T = int8_t storage holding unsigned bytes, int32 C holding the uint32 product): the MFMA is
// signed only, so each fragment's bytes are flipped to s = u - 128 (XOR 0x80) before the first
// MFMA that reads it, and the lane adds its fragments' signed bytes (v_dot4 against ones) into
// per-row and per-column sums RA, CB.  Per k position u_a u_b = s_a s_b + 128 (s_a + s_b) + 16384,
// so C = A_s B_s + 128 (RA[m] + CB[n]) + 16384 Kp, all modulo 2^32 -- exactly the uint32-wrapped
// unsigned product.  Kp counts every k position the kernel accumulated, the zero padding of a
// ragged K too: a padded position has u = 0, s = -128 on both sides and adds 16384 - 32768 +
// 16384 = 0 to the identity.
template <typename T, typename OutT, bool EPI, bool RAGGED, bool AK, bool BK, bool U8 = false>
__global__ void __launch_bounds__(256, 1)
    gemm_tn16_kernel(const T* __restrict__ A, const T* __restrict__ B, OutT* __restrict__ C, int tiles_m, int tiles_n,
                     int ktiles, int64_t lda_b, int64_t ldb_b, int64_t ldc, Epilogue epi, TnBounds bnd) {
    static_assert(!U8 || (std::is_same<T, int8_t>::value && !EPI), "U8: bytes in int8_t storage, plain int32 output");
    using AccV = typename Mfma16<T>::acc_t;
    typedef typename Mfma16<T>::acc_elem Acc;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * 2 * TN_SLICE];  // [stage][A,B][32 KB]

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int tm, tn;
    xcd_tile(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
    const int wm = w >> 1, wn = w & 1;
    const int h = lane >> 5;

    // Rows (m, n) of this tile inside the matrix: all 256 unless RAGGED and the tile is the last.
    int a_rows = TN_TILE, b_rows = TN_TILE;
    if constexpr (RAGGED) {
        a_rows = (int)(bnd.m - (int64_t)tm * TN_TILE < TN_TILE ? bnd.m - (int64_t)tm * TN_TILE : TN_TILE);
        b_rows = (int)(bnd.n - (int64_t)tn * TN_TILE < TN_TILE ? bnd.n - (int64_t)tn * TN_TILE : TN_TILE);
    }
    const int kelems = bnd.kb / (int)sizeof(T);
    TnSide<T, AK> sa;
    TnSide<T, BK> sb;
    sa.init(A, lda_b, tm, a_rows, bnd.m, kelems, w, wm, lane);
    sb.init(B, ldb_b, tn, b_rows, bnd.n, kelems, w, wn, lane);
    // wave w fills 8 KB of each slice: K-contiguous rows [64 w, 64 w + 64), M/N-contiguous
    // k rows [16 w, 16 w + 16); instruction i 1 KB of it
    const uint32_t lds0 = lds_addr(smem) + w * 64 * TN_KB;

    // DMA load q (0..15) of a k-tile into `stage`: q < 8 are A, q >= 8 B.
    auto dma = [&](int q, int stage, uint32_t kofs) {
        const int i = q & 7;
        const uint32_t dst = lds0 + stage * 2 * TN_SLICE + (q >> 3) * TN_SLICE + i * 1024;
        if (q < 8) {
            uint32_t off = sa.voff(i);
            if constexpr (RAGGED) off = sa.valid(i, kofs, bnd.kb) ? off : OOB_OFS;
            dma16(sa.rs, off, sa.soff(i, kofs), dst);
        } else {
            uint32_t off = sb.voff(i);
            if constexpr (RAGGED) off = sb.valid(i, kofs, bnd.kb) ? off : OOB_OFS;
            dma16(sb.rs, off, sb.soff(i, kofs), dst);
        }
    };

    AccV acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0;

    // ---- fragments: 16x16 MFMA operands, 16 bytes per lane: row (m or n) lane % 16 of a
    // 16-row block, 8 k values (16-bit) or 16 (int8) at 8 (lane / 16) of k-step u (the
    // 64-byte half u of the stage's 128 bytes of K).  a[i]: rows 16 i of the wave's 128 m;
    // b[j]: rows 16 j of its 128 n.
    struct F16 {
        uint4 a[8], b[8];
    };
    // fragment t (0..15) of k-step u, in the order the MFMAs (i-major) first use them:
    // a[0], b[0..7], a[1..7]
    auto rd16 = [&](F16& f, const uint8_t* stage, int u, int t) {
        const bool isa = t == 0 || t > 8;
        const int blk = t == 0 ? 0 : (t <= 8 ? t - 1 : t - 8);
        if (isa) f.a[blk] = sa.read16(stage, u, blk);
        else f.b[blk] = sb.read16(stage + TN_SLICE, u, blk);
    };
    // MFMA A operand = B fragment (rows are columns n of C), B operand = A fragment (rows
    // m): acc[i][j] register r of lane l is C[m][n], m = 128 wm + 16 i + l % 16,
    // n = 128 wn + 16 j + 4 (l / 16) + r.

    // Per k-tile kt (stage kt % 2), one barrier, at the middle:
    //   first half:  64 MFMAs of k-step 0 (fragments read during the previous tile); the
    //                16 fragment reads of k-step 1 from this stage, one per 4 MFMAs;
    //   middle:      this wave's DMAs of tile kt + 1 (issued during the previous tile's
    //                second half) landed; barrier: tile kt + 1 published, and every read
    //                of this stage done;
    //   second half: 64 MFMAs of k-step 1; tile kt + 1's k-step 0 reads from the other
    //                stage and the DMAs of tile kt + 2 into this one, each one per 4 MFMAs.
    // A DMA thus has about a whole k-tile to land.  Past the last tile the DMAs re-fetch
    // the last one into the idle stage.
#pragma unroll
    for (int q = 0; q < 16; ++q) dma(q, 0, 0);
#pragma unroll
    for (int q = 0; q < 16; ++q) dma(q, 1, ktiles > 1 ? (uint32_t)TN_KB : 0u);
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");   // tile 0 (the first 16 of this wave's loads)
    __syncthreads();
    F16 fa, fb;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        rd16(fa, smem, 0, t);
        __builtin_amdgcn_sched_barrier(0);
    }
    // U8: signed-byte sums of this wavefront's A rows (ra[i]: row 16 i + lane % 16 of its 128) and
    // B columns (rb[j]), over the k bytes of this lane's 16-lane group
    int32_t ra[8], rb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ra[i] = rb[i] = 0;
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
    // fragment t in read order (a[0], b[0..7], a[1..7]).  Each is flipped two reads after its own
    // read was issued, well before its first MFMA, so that neither the LDS latency nor the
    // VALU-to-MFMA wait sits in front of an MFMA; the last two of a k-step are flipped early in
    // the next one (their first MFMAs come at 48 and 56).  Fragments read past the last k-tile
    // are never flipped, so they do not enter the sums.
    auto flip_t = [&](F16& f, int t) __attribute__((always_inline)) {
        if constexpr (U8) {
            if (t == 0) flip(f.a[0], ra[0]);
            else if (t <= 8) flip(f.b[t - 1], rb[t - 1]);
            else flip(f.a[t - 8], ra[t - 8]);
        }
    };
#pragma unroll
    for (int t = 0; t < 16; ++t) flip_t(fa, t);

    for (int kt = 0; kt < ktiles; ++kt) {
        const int st = kt & 1;
        const uint8_t* base = smem + st * 2 * TN_SLICE;
        const uint8_t* next = smem + (st ^ 1) * 2 * TN_SLICE;
        const uint32_t kofs2 = (uint32_t)(kt + 2 < ktiles ? kt + 2 : ktiles - 1) * TN_KB;
#pragma unroll
        for (int q = 0; q < 64; ++q) {
            acc[q >> 3][q & 7] = Mfma16<T>::run(fa.b[q & 7], fa.a[q >> 3], acc[q >> 3][q & 7]);
            if ((q & 3) == 3) rd16(fb, base, 1, q >> 2);
            if ((q == 2 || q == 6) && kt > 0) flip_t(fa, 14 + (q >> 2));
            if ((q & 3) == 3 && (q >> 2) >= 2) flip_t(fb, (q >> 2) - 2);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's part of tile kt + 1 landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 64; ++q) {
            acc[q >> 3][q & 7] = Mfma16<T>::run(fb.b[q & 7], fb.a[q >> 3], acc[q >> 3][q & 7]);
            if ((q & 3) == 1) rd16(fa, next, 0, q >> 2);
            if ((q & 3) == 3) dma(q >> 2, st, kofs2);
            if (q == 2 || q == 6) flip_t(fb, 14 + (q >> 2));
            if ((q & 3) == 3 && (q >> 2) >= 2 && kt + 1 < ktiles) flip_t(fa, (q >> 2) - 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- epilogue through LDS, so that global stores are whole 512-byte row runs.
    // acc[I][j] register r of lane l is C[m][n] with m = 128 wm + 16 I + l % 16 and
    // n = 128 wn + 16 j + 4 (l / 16) + r within the tile (the 16x16 MFMA accumulator
    // map, I and j = 0..7).  Each wave stages 32 rows x 128 columns at a time (a row
    // quarter i: I = 2 i, 2 i + 1) in its own 16.5 KB of the idle stage buffers (4 waves:
    // 66 KB of the 128 KB), rows padded to 528 bytes so the 32 rows of one column group
    // land on distinct banks; then reads whole rows back: lanes 0..31 and 32..63 each
    // cover one 512-byte row per instruction.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    constexpr int EP_PITCH = 128 * 4 + 16;
    if constexpr (U8) {
        // full sums: the four 16-lane groups hold the four 16-byte quarters of every k-step
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ra[i] += __shfl_xor(ra[i], 16, 64);
            ra[i] += __shfl_xor(ra[i], 32, 64);
            rb[i] += __shfl_xor(rb[i], 16, 64);
            rb[i] += __shfl_xor(rb[i], 32, 64);
        }
        // acc[i][j] register r: row 16 i + lane % 16 (this lane's ra[i]), column 16 j + 4 (lane / 16) + r
        // (rb[j] of lane 4 (lane / 16) + r)
        const uint32_t kconst = 16384u * (uint32_t)ktiles * (uint32_t)TN_KB;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t cb[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) cb[r] = (uint32_t)__shfl(rb[j], 4 * (lane >> 4) + r, 64);
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[i][j][r] = (int32_t)((uint32_t)acc[i][j][r] + 128u * ((uint32_t)ra[i] + cb[r]) + kconst);
        }
    }

    const int rr = lane & 31;
    uint8_t* ep = smem + w * (32 * EP_PITCH);
    typedef Acc Acc4 __attribute__((ext_vector_type(4)));
    const int64_t row0 = (int64_t)tm * TN_TILE + wm * 128, col0 = (int64_t)tn * TN_TILE + wn * 128;
    OutT* cbase = C + row0 * ldc + col0;
    // columns of this lane's 4-column group inside the matrix (RAGGED: 0..4)
    int cols_in = 4;
    if constexpr (RAGGED) {
        const int64_t left = bnd.n - (col0 + 4 * rr);
        cols_in = left >= 4 ? 4 : (left > 0 ? (int)left : 0);
    }
    // one row quarter i at a time; i is a template constant so that acc stays in registers
    typedef float F4 __attribute__((ext_vector_type(4)));
    auto quarter = [&](auto itag) {
        constexpr int i = decltype(itag)::value;
        // The epilogue's init terms for the 16 rows x 4 columns this lane finishes, all
        // requested before the staging so that their HBM latency overlaps it (loaded one
        // row at a time inside the store loop they cost one round trip per row).
        F4 rin[EPI ? 16 : 1];
        float bin[EPI ? 16 : 1];
        F4 bcol = {0.f, 0.f, 0.f, 0.f};
        if constexpr (EPI) {
            const int64_t n = col0 + 4 * rr;
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
            for (int t = 0; t < 16; ++t) {
                const int64_t m = row0 + 32 * i + 2 * t + h;
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
            for (int j = 0; j < 8; ++j) {
                const Acc4 v = {acc[2 * i + ii][j][0], acc[2 * i + ii][j][1], acc[2 * i + ii][j][2], acc[2 * i + ii][j][3]};
                *reinterpret_cast<Acc4*>(ep + (16 * ii + (lane & 15)) * EP_PITCH + (16 * j + 4 * (lane >> 4)) * 4) = v;
            }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's staged rows are in LDS
        __builtin_amdgcn_wave_barrier();
        auto store_rows = [&](auto acttag) {
            constexpr int ACT = decltype(acttag)::value;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int row = 2 * t + h;                       // 0..31 of this i
                const Acc4 v = *reinterpret_cast<const Acc4*>(ep + row * EP_PITCH + rr * 16);
                OutT* dst = cbase + (int64_t)(32 * i + row) * ldc + 4 * rr;
                if (RAGGED && row0 + 32 * i + row >= bnd.m) continue;
                if constexpr (!EPI && std::is_same<OutT, Acc>::value) {
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
                        float x = (float)v[k];
                        // the same fp32 sums as epi_apply: (bias + residual), then acc + that
                        if constexpr (EPI) x = epi_act_c<ACT>(x + ((bin[t] + bcol[k]) + rin[t][k]));
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
            switch (epi.act) {   // uniform: one branch per quarter, none per element
            case EPI_RELU: store_rows(std::integral_constant<int, EPI_RELU>{}); break;
            case EPI_GELU_TANH: store_rows(std::integral_constant<int, EPI_GELU_TANH>{}); break;
            case EPI_GELU_ERF: store_rows(std::integral_constant<int, EPI_GELU_ERF>{}); break;
            default: store_rows(std::integral_constant<int, EPI_NONE>{}); break;
            }
        } else {
            store_rows(std::integral_constant<int, EPI_NONE>{});
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);   // reads done before the next i overwrites
        __builtin_amdgcn_wave_barrier();
    };
    quarter(std::integral_constant<int, 0>{});
    quarter(std::integral_constant<int, 1>{});
    quarter(std::integral_constant<int, 2>{});
    quarter(std::integral_constant<int, 3>{});
}


// Which kernel applies (see TnFit): the operand forms AK (A K-contiguous, i.e. row-major)
// and BK (B K-contiguous, i.e. column-major).
template <typename T>
int tn_gemm_eligible(const void* A, const void* B, const void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                     int64_t ldb, int64_t ldc, size_t c_elem, bool ak, bool bk) {
    const int64_t sz = (int64_t)sizeof(T), ke = TN_KB / sz, chunk = 16 / sz;
    if (M <= 0 || N <= 0 || K <= 0) return TN_NO;
    if ((ak || bk) && K % chunk) return TN_NO;           // a K-contiguous chunk wholly in or out
    if ((!ak && M % chunk) || (!bk && N % chunk)) return TN_NO;
    const int64_t tiles_m = (M + TN_TILE - 1) / TN_TILE, tiles_n = (N + TN_TILE - 1) / TN_TILE;
    if (tiles_m * tiles_n > 0x7fffffff || (K + ke - 1) / ke > 0x7fffffff || K * sz > 0x7fffffff) return TN_NO;
    if ((lda * sz) % 16 || (ldb * sz) % 16 || !aligned(A, 16) || !aligned(B, 16)) return TN_NO;
    // buffer offsets are 32-bit: a 256-row K-contiguous slab, or the whole K x ld
    // M/N-contiguous operand, must span < 2 GiB
    const int64_t lim = (int64_t)1 << 31;
    if ((ak ? (int64_t)TN_TILE * lda * sz : K * lda * sz) >= lim) return TN_NO;
    if ((bk ? (int64_t)TN_TILE * ldb * sz : K * ldb * sz) >= lim) return TN_NO;
    if (M % TN_TILE == 0 && N % TN_TILE == 0 && K % ke == 0 && ldc % 4 == 0 && aligned(C, 4 * c_elem))
        return TN_FULL;
    // ragged: worth the 256 x 256 tiles once the product is no longer launch-bound
    return M * N >= (int64_t)TN_TILE * TN_TILE ? TN_RAGGED : TN_NO;
}

template <typename T, typename OutT, bool EPI, bool AK, bool BK, bool U8 = false>
int launch_gemm_tn_layout(const T* A, const T* B, OutT* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                          int64_t ldc, hipStream_t s, const Epilogue& epi, bool ragged) {
    const int tiles_m = (int)((M + TN_TILE - 1) / TN_TILE), tiles_n = (int)((N + TN_TILE - 1) / TN_TILE);
    const int64_t ke = TN_KB / (int64_t)sizeof(T);
    const int ktiles = (int)((K + ke - 1) / ke);
    TnBounds bnd;
    bnd.m = M;
    bnd.n = N;
    bnd.kb = (int)(K * (int64_t)sizeof(T));
    bnd.cvec = ldc % 4 == 0 && aligned(C, 4 * sizeof(OutT));
    const int64_t lda_b = lda * (int64_t)sizeof(T), ldb_b = ldb * (int64_t)sizeof(T);
    if (ragged)
        hipLaunchKernelGGL((gemm_tn16_kernel<T, OutT, EPI, true, AK, BK, U8>), dim3((unsigned)(tiles_m * tiles_n)),
                           dim3(256), 0, s, A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd);
    else
        hipLaunchKernelGGL((gemm_tn16_kernel<T, OutT, EPI, false, AK, BK, U8>), dim3((unsigned)(tiles_m * tiles_n)),
                           dim3(256), 0, s, A, B, C, tiles_m, tiles_n, ktiles, lda_b, ldb_b, ldc, epi, bnd);
    LAVA_LAUNCH_CHECK("gemm_tn_kernel");
    return LAVA_HIP_OK;
}

// Instantiations live in one translation unit per operand form (they compile in parallel).
#define LAVA_TN_LAYOUT_INST(T, O, E, AK, BK)                                                                        \
    template int launch_gemm_tn_layout<T, O, E, AK, BK>(const T*, const T*, O*, int64_t, int64_t, int64_t, int64_t, \
                                                        int64_t, int64_t, hipStream_t, const Epilogue&, bool);
#define LAVA_TN_LAYOUT_EXTERN(T, O, E, AK, BK)                                                                        \
    extern template int launch_gemm_tn_layout<T, O, E, AK, BK>(const T*, const T*, O*, int64_t, int64_t, int64_t,   \
                                                               int64_t, int64_t, int64_t, hipStream_t,                \
                                                               const Epilogue&, bool);
// The unsigned 8-bit instance of one operand form (bytes in int8_t storage, uint32 product in int32).
#define LAVA_TN_LAYOUT_U8_INST(AK, BK)                                                                              \
    template int launch_gemm_tn_layout<int8_t, int32_t, false, AK, BK, true>(                                     \
        const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, hipStream_t, \
        const Epilogue&, bool);
#define LAVA_TN_LAYOUT_U8_EXTERN(AK, BK)                                                                            \
    extern template int launch_gemm_tn_layout<int8_t, int32_t, false, AK, BK, true>(                              \
        const int8_t*, const int8_t*, int32_t*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, hipStream_t, \
        const Epilogue&, bool);
// The 16-bit set of one operand form: plain fp32 output, and the epilogue to fp32 / fp16 / bf16.
#define LAVA_TN_LAYOUT_16BIT(M, AK, BK) \
    M(f16, float, false, AK, BK)        \
    M(bf16, float, false, AK, BK)       \
    M(f16, float, true, AK, BK)         \
    M(f16, f16, true, AK, BK)           \
    M(f16, bf16, true, AK, BK)          \
    M(bf16, float, true, AK, BK)        \
    M(bf16, f16, true, AK, BK)          \
    M(bf16, bf16, true, AK, BK)

}  // namespace lava
