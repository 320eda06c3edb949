// lava_coopmat.hpp -- the cooperative-matrix device vocabulary on CDNA4 (gfx950).
//
// Lava.jl's kernels are written against an opaque subgroup tile,
// `CoopMatrix{T,M,N,Use,Scope}` (src/vocabulary/coopmat.jl:36-92), and eleven
// operations on it (src/vocabulary/coopmat.jl:216-312).  On MI355X a subgroup is a
// 64-lane wavefront and the tile lives in the registers an MFMA instruction reads
// and writes, so the "opaque handle" becomes `Frag<T, R, C, Use>`: the lane's share
// of an R x C tile, held as a small array of registers whose (row, column) mapping
// is the MFMA operand layout below.
//
// Layouts (64 lanes, lane = threadIdx.x % 64):
//   Accumulator R x C, C in {16, 32}:
//     C == 16: lane holds column lane % 16, rows 4 * (lane / 16) + j,            j < 4
//     C == 32: lane holds column lane % 32, rows 8 * (j / 4) + 4 * (lane / 32) + j % 4,
//              j < 16
//   MatrixA R x K, R in {16, 32}: lane holds row lane % R, columns (k)
//     (lane / R) * (K * R / 64) + j, j < K * R / 64 -- consecutive k per lane.
//   MatrixB K x C, C in {16, 32}: lane holds column lane % C, rows (k)
//     (lane / C) * (K * C / 64) + j.
// A and B share one k distribution, and an MFMA pairs A's slot (group, j) with
// B's slot (group, j), so the product is the same whatever order the hardware
// consumes the slots in; the accumulator map is the one fact taken from the
// hardware, and the per-element identity test pins it.
//
// Semantics of each operation are those of the SPIR-V instruction Lava's emitter
// writes for it (src/compiler/spirv/coopmat.jl:664-991):
//   load / store          OpCooperativeMatrixLoad/StoreKHR, ColumnMajor by default,
//                         RowMajor on request (coopmat.jl:664-744).  Offsets here are
//                         0-based element offsets; the host mirror maps Lava's 1-based
//                         `offset` onto them (src/device/coopmat_intrinsics.jl:57-75).
//   zero                  OpConstantNull (coopmat.jl:746-762)
//   mma                   OpCooperativeMatrixMulAddKHR; int8 operands signed
//                         (coopmat.jl:115-151, 764-781)
//   convert               OpFConvert, round to nearest even (coopmat.jl:783-824;
//                         src/compiler/passes/exact_narrowing.jl:31-36)
//   mul / add             OpFMul / OpFAdd component-wise (coopmat.jl:870-885)
//   length/getcomp/setcomp  this lane's components, 0-based (coopmat.jl:826-868)
//   perelement            OpCooperativeMatrixPerElementOpNV: f(row, col, e, extras...)
//                         with 0-based row/col (src/device/coopmat_intrinsics.jl:535-678)
//   reduce                OpCooperativeMatrixReduceNV: combine along Row (1), Column
//                         (2) or both (3); the result is smeared over the reduced
//                         axis, not a vector (src/device/coopmat_intrinsics.jl:685-755);
//                         reduce_into: the same into a destination of another extent,
//                         and the TwoByTwo (4) block form
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lava {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Vectors in LDS: the components packed, aligned to 2x (2 components) or 4x
// (4 components) the component -- the layout Lava's emitter gives `@localmem`
// vectors (src/compiler/spirv/types.jl:838-900, test_workgroup_vector_layout.jl:24-27).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
static_assert(sizeof(f16x2) == 4 && alignof(f16x2) == 4, "<2 x half> in LDS: 4 bytes, align 4");
static_assert(sizeof(f16x4) == 8 && alignof(f16x4) == 8, "<4 x half> in LDS: 8 bytes, align 8");
static_assert(sizeof(f32x2) == 8 && alignof(f32x2) == 8, "<2 x float> in LDS: 8 bytes, align 8");
static_assert(sizeof(f32x4) == 16 && alignof(f32x4) == 16, "<4 x float> in LDS: 16 bytes, align 16");

enum Use { MatrixA = 0, MatrixB = 1, Accumulator = 2 };

// CoopMatReduce masks (src/vocabulary/coopmat.jl:292-297)
enum ReduceMask : uint32_t { ReduceRow = 1u, ReduceColumn = 2u, ReduceRowAndColumn = 3u, ReduceTwoByTwo = 4u };

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

// ---------------------------------------------------------------------------
// Lane <-> (row, col) maps
// ---------------------------------------------------------------------------
template <int R, int C, Use U>
struct Layout;

template <int R, int K>
struct Layout<R, K, MatrixA> {
    static_assert(R == 16 || R == 32, "MatrixA rows must be 16 or 32");
    static constexpr int groups = 64 / R;
    static constexpr int len = K / groups;
    static_assert(len * groups == K && len >= 1, "K must split over the lane groups");
    __host__ __device__ static constexpr int row(int lane, int) { return lane % R; }
    __host__ __device__ static constexpr int col(int lane, int j) { return (lane / R) * len + j; }
};

template <int K, int C>
struct Layout<K, C, MatrixB> {
    static_assert(C == 16 || C == 32, "MatrixB columns must be 16 or 32");
    static constexpr int groups = 64 / C;
    static constexpr int len = K / groups;
    static_assert(len * groups == K && len >= 1, "K must split over the lane groups");
    __host__ __device__ static constexpr int row(int lane, int j) { return (lane / C) * len + j; }
    __host__ __device__ static constexpr int col(int lane, int) { return lane % C; }
};

template <>
struct Layout<16, 16, Accumulator> {
    static constexpr int len = 4;
    __host__ __device__ static constexpr int row(int lane, int j) { return 4 * (lane / 16) + j; }
    __host__ __device__ static constexpr int col(int lane, int) { return lane % 16; }
};

// Accumulators of other extents (coopmat2's flexible dimensions, used by a reduce into a
// destination of another shape): R x C with R and C multiples of 16, as (R / 16) x (C / 16)
// sub-tiles of the 16 x 16 map in row-major order -- slot j is sub-tile j / 4, row
// 4 (lane / 16) + j % 4 and column lane % 16 within it.  (32 x 32 keeps the 32x32x16 MFMA's map.)
template <int R, int C>
struct Layout<R, C, Accumulator> {
    static_assert(R % 16 == 0 && C % 16 == 0 && R >= 16 && C >= 16, "Accumulator extents are multiples of 16");
    static constexpr int tc = C / 16;
    static constexpr int len = R * C / 64;
    __host__ __device__ static constexpr int row(int lane, int j) { return 16 * ((j / 4) / tc) + 4 * (lane / 16) + j % 4; }
    __host__ __device__ static constexpr int col(int lane, int j) { return 16 * ((j / 4) % tc) + lane % 16; }
};

// The 8 x 8 result of a TwoByTwo reduce of a 16 x 16 tile: one element per lane.
template <>
struct Layout<8, 8, Accumulator> {
    static constexpr int len = 1;
    __host__ __device__ static constexpr int row(int lane, int) { return lane / 8; }
    __host__ __device__ static constexpr int col(int lane, int) { return lane % 8; }
};

template <>
struct Layout<32, 32, Accumulator> {
    static constexpr int len = 16;
    __host__ __device__ static constexpr int row(int lane, int j) { return 8 * (j / 4) + 4 * (lane / 32) + (j % 4); }
    __host__ __device__ static constexpr int col(int lane, int) { return lane % 32; }
};

// ---------------------------------------------------------------------------
// Fragment
// ---------------------------------------------------------------------------
template <typename T, int R, int C, Use U>
struct Frag {
    using L = Layout<R, C, U>;
    static constexpr int len = L::len;
    T v[L::len];
};

// coopmat_length / getcomp / setcomp.  length is a property of the type (how the
// MFMA layout splits R x C over 64 lanes: R * C / 64 components per lane); the
// component index is 0-based and names this lane's slot j of the layout above.
template <typename FragT>
__host__ __device__ __forceinline__ constexpr int length() { return FragT::len; }
template <typename T, int R, int C, Use U>
__device__ __forceinline__ constexpr int length(const Frag<T, R, C, U>&) { return Frag<T, R, C, U>::len; }
template <typename T, int R, int C, Use U>
__device__ __forceinline__ T getcomp(const Frag<T, R, C, U>& m, int i) { return m.v[i]; }
template <typename T, int R, int C, Use U>
__device__ __forceinline__ Frag<T, R, C, U> setcomp(Frag<T, R, C, U> m, int i, T x) { m.v[i] = x; return m; }

template <typename FragT>
__device__ __forceinline__ FragT zero() {
    FragT m;
#pragma unroll
    for (int j = 0; j < FragT::len; ++j) m.v[j] = 0;
    return m;
}

// Element (r, c) of a tile whose top-left is p: row-major r*ld + c, column-major
// c*ld + r.  `ld` is Lava's `stride`, the distance between consecutive columns
// (column-major) or rows (row-major), in elements.
__device__ __forceinline__ int64_t tile_index(int r, int c, int64_t ld, bool rowmajor) {
    return rowmajor ? (int64_t)r * ld + c : (int64_t)c * ld + r;
}

template <typename FragT, typename S>
__device__ __forceinline__ FragT load(const S* p, int64_t ld, bool rowmajor) {
    FragT m;
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < FragT::len; ++j)
        m.v[j] = (decltype(m.v[0]))p[tile_index(FragT::L::row(lane, j), FragT::L::col(lane, j), ld, rowmajor)];
    return m;
}

template <typename S, typename T, int R, int C, Use U>
__device__ __forceinline__ void store(S* p, int64_t ld, bool rowmajor, const Frag<T, R, C, U>& m) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < Frag<T, R, C, U>::len; ++j)
        p[tile_index(Frag<T, R, C, U>::L::row(lane, j), Frag<T, R, C, U>::L::col(lane, j), ld, rowmajor)] = (S)m.v[j];
}

// ---------------------------------------------------------------------------
// Round-to-nearest-even narrowing (coopmat_convert of an fp32 accumulator)
// ---------------------------------------------------------------------------
template <typename To>
__device__ __forceinline__ To narrow(float x);
template <>
__device__ __forceinline__ float narrow<float>(float x) { return x; }
template <>
__device__ __forceinline__ f16 narrow<f16>(float x) { return (f16)x; }     // v_cvt_f16_f32, RNE
template <>
__device__ __forceinline__ bf16 narrow<bf16>(float x) { return (bf16)x; }  // v_cvt_pk_bf16_f32, RNE

template <typename To, typename T, int R, int C, Use U>
__device__ __forceinline__ Frag<To, R, C, U> convert(const Frag<T, R, C, U>& m) {
    Frag<To, R, C, U> o;
#pragma unroll
    for (int j = 0; j < Frag<T, R, C, U>::len; ++j) o.v[j] = narrow<To>((float)m.v[j]);
    return o;
}

// Whether two uses of an R x C tile put every element in the same lane and slot.
// True for a 16 x 16 Accumulator and a 16 x 16 MatrixB (K = 16): both hold column
// lane % 16, rows 4 (lane / 16) + j.
template <int R, int C, Use U1, Use U2>
__host__ __device__ constexpr bool same_lane_map() {
    using L1 = Layout<R, C, U1>;
    using L2 = Layout<R, C, U2>;
    if (L1::len != L2::len) return false;
    for (int lane = 0; lane < 64; ++lane)
        for (int j = 0; j < L1::len; ++j)
            if (L1::row(lane, j) != L2::row(lane, j) || L1::col(lane, j) != L2::col(lane, j)) return false;
    return true;
}

// LDS traffic of one wavefront is performed in issue order; the fence (lgkmcnt(0)
// and a compiler barrier) orders this lane's LDS stores before the other lanes'
// loads that follow.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    __builtin_amdgcn_wave_barrier();
}

// coopmat_convert with a change of use, e.g. an fp32 Accumulator to an fp16 MatrixA
// (the P operand of attention's second product; OpFConvert then
// OpCooperativeMatrixConvertNV, src/compiler/spirv/coopmat.jl:783-824;
// src/device/coopmat_intrinsics.jl:222-247).  The component type is narrowed first
// (RNE), at the source use, as the emitter does.  Where both uses map elements to
// the same lanes the relayout is free; otherwise the tile goes through `scratch`, R x C
// elements of LDS private to this wavefront: each lane stores its components at
// (row, col) and loads the destination use's (row, col).
template <typename To, Use UTo, typename T, int R, int C, Use U>
__device__ __forceinline__ Frag<To, R, C, UTo> convert(const Frag<T, R, C, U>& m, To* scratch) {
    Frag<To, R, C, UTo> o;
    if constexpr (same_lane_map<R, C, U, UTo>()) {
#pragma unroll
        for (int j = 0; j < Frag<T, R, C, U>::len; ++j) o.v[j] = narrow<To>((float)m.v[j]);
    } else {
        using LS = Layout<R, C, U>;
        using LD = Layout<R, C, UTo>;
        const int lane = lane_id();
        wave_lds_sync();   // earlier reads of scratch by other lanes are done
#pragma unroll
        for (int j = 0; j < LS::len; ++j) scratch[LS::row(lane, j) * C + LS::col(lane, j)] = narrow<To>((float)m.v[j]);
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < LD::len; ++j) o.v[j] = scratch[LD::row(lane, j) * C + LD::col(lane, j)];
    }
    return o;
}

// coopmat_mul / coopmat_add: OpFMul / OpFAdd, component-wise
// (src/compiler/spirv/coopmat.jl:870-885).  With one operand loaded at stride 0 (every
// column reads the same vector) mul is the per-row rescale and add the bias of
// `accinit` (src/device/coopmat_intrinsics.jl:402-464).
template <typename T, int R, int C, Use U>
__device__ __forceinline__ Frag<T, R, C, U> mul(const Frag<T, R, C, U>& a, const Frag<T, R, C, U>& b) {
    Frag<T, R, C, U> o;
#pragma unroll
    for (int j = 0; j < Frag<T, R, C, U>::len; ++j) o.v[j] = a.v[j] * b.v[j];
    return o;
}
template <typename T, int R, int C, Use U>
__device__ __forceinline__ Frag<T, R, C, U> add(const Frag<T, R, C, U>& a, const Frag<T, R, C, U>& b) {
    Frag<T, R, C, U> o;
#pragma unroll
    for (int j = 0; j < Frag<T, R, C, U>::len; ++j) o.v[j] = a.v[j] + b.v[j];
    return o;
}

// ---------------------------------------------------------------------------
// coopmat_perelement: f(row, col, e, extras...) with 0-based row and col
// ---------------------------------------------------------------------------
template <typename F, typename T, int R, int C, Use U, typename... X>
__device__ __forceinline__ Frag<T, R, C, U> perelement(F f, Frag<T, R, C, U> m, X... extras) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < Frag<T, R, C, U>::len; ++j)
        m.v[j] = f((uint32_t)Frag<T, R, C, U>::L::row(lane, j), (uint32_t)Frag<T, R, C, U>::L::col(lane, j), m.v[j],
                   extras...);
    return m;
}

// The matrix-operand form: f(row, col, m_e, o_e) over corresponding elements.
template <typename F, typename T, int R, int C, Use U>
__device__ __forceinline__ Frag<T, R, C, U> perelement_m(F f, Frag<T, R, C, U> m, const Frag<T, R, C, U>& o) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < Frag<T, R, C, U>::len; ++j)
        m.v[j] = f((uint32_t)Frag<T, R, C, U>::L::row(lane, j), (uint32_t)Frag<T, R, C, U>::L::col(lane, j), m.v[j],
                   o.v[j]);
    return m;
}

// ---------------------------------------------------------------------------
// Cross-lane exchange (ds_swizzle-free: ds_bpermute through __shfl_xor)
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T xor_lane(T x, int mask) {
    static_assert(sizeof(T) == 4, "32-bit lanes only");
    return __shfl_xor(x, mask, 64);
}

// coopmat_reduce over an accumulator fragment, same-shape destination.
// Row: combine the elements of each row (across columns); Column: of each column.
template <uint32_t MASK, typename F, typename T, int R, int C>
__device__ __forceinline__ Frag<T, R, C, Accumulator> reduce(F f, Frag<T, R, C, Accumulator> m) {
    constexpr int ncol_lanes = C;  // lanes sharing a row differ in lane % C
    if constexpr ((MASK & ReduceRow) != 0) {
#pragma unroll
        for (int j = 0; j < Frag<T, R, C, Accumulator>::len; ++j) {
#pragma unroll
            for (int s = 1; s < ncol_lanes; s <<= 1) m.v[j] = f(m.v[j], xor_lane(m.v[j], s));
        }
    }
    if constexpr ((MASK & ReduceColumn) != 0) {
        T acc = m.v[0];
#pragma unroll
        for (int j = 1; j < Frag<T, R, C, Accumulator>::len; ++j) acc = f(acc, m.v[j]);
#pragma unroll
        for (int s = ncol_lanes; s < 64; s <<= 1) acc = f(acc, xor_lane(acc, s));
#pragma unroll
        for (int j = 0; j < Frag<T, R, C, Accumulator>::len; ++j) m.v[j] = acc;
    }
    return m;
}

// coopmat_reduce into a destination of another extent (OpCooperativeMatrixReduceNV with coopmat2
// flexible dimensions; src/device/coopmat_intrinsics.jl:685-720: the reference's smearReduce
// resizes a Br x Bc matrix to Br x HSV_pad).  Row: Dst has m's rows and any number of columns,
// every column of row r holding row r's combination; Column: m's columns, any rows; RowAndColumn:
// any extent, every element the combination of all of m; TwoByTwo: Dst is (R / 2) x (C / 2),
// element (i, j) = f(f(m[2i][2j], m[2i][2j+1]), f(m[2i+1][2j], m[2i+1][2j+1])) -- the 2 x 2 block
// reduce of the published SPV_NV_cooperative_matrix2 extension (the reference ships the mask bit
// unverified), combined in that order.  The values cross lanes through `lds` (R * C elements of
// the calling wavefront's workgroup memory); every lane of the wavefront calls it.
template <uint32_t MASK, int RD, int CD, typename F, typename T, int R, int C>
__device__ __forceinline__ Frag<T, RD, CD, Accumulator> reduce_into(F f, const Frag<T, R, C, Accumulator>& m,
                                                                     T* lds) {
    using LS = Layout<R, C, Accumulator>;
    using LD = Layout<RD, CD, Accumulator>;
    const int lane = lane_id();
    Frag<T, RD, CD, Accumulator> d;
    if constexpr (MASK == ReduceTwoByTwo) {
        static_assert(2 * RD == R && 2 * CD == C, "a TwoByTwo reduce halves both extents");
#pragma unroll
        for (int j = 0; j < LS::len; ++j) lds[LS::row(lane, j) * C + LS::col(lane, j)] = m.v[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < LD::len; ++j) {
            const int i = LD::row(lane, j), k = LD::col(lane, j);
            const T* b = lds + (2 * i) * C + 2 * k;
            d.v[j] = f(f(b[0], b[1]), f(b[C], b[C + 1]));
        }
    } else {
        static_assert(MASK >= 1u && MASK <= 3u, "Row, Column, RowAndColumn or TwoByTwo");
        static_assert((MASK & ReduceRow) == 0 || (MASK & ReduceColumn) != 0 || RD == R,
                      "a Row reduce keeps the rows");
        static_assert((MASK & ReduceColumn) == 0 || (MASK & ReduceRow) != 0 || CD == C,
                      "a Column reduce keeps the columns");
        const auto sm = reduce<MASK>(f, m);   // same shape, smeared
#pragma unroll
        for (int j = 0; j < LS::len; ++j) lds[LS::row(lane, j) * C + LS::col(lane, j)] = sm.v[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < LD::len; ++j) {
            const int r = MASK == ReduceRow ? LD::row(lane, j) : 0;
            const int c = MASK == ReduceColumn ? LD::col(lane, j) : 0;
            d.v[j] = lds[r * C + c];
        }
    }
    return d;
}

// ---------------------------------------------------------------------------
// coopmat_muladd: D = A * B + C, accumulated in C's type
// ---------------------------------------------------------------------------
__device__ __forceinline__ Frag<float, 16, 16, Accumulator> mma(const Frag<f16, 16, 16, MatrixA>& a,
                                                                const Frag<f16, 16, 16, MatrixB>& b,
                                                                Frag<float, 16, 16, Accumulator> c) {
    f16x4 av = {a.v[0], a.v[1], a.v[2], a.v[3]};
    f16x4 bv = {b.v[0], b.v[1], b.v[2], b.v[3]};
    f32x4 cv = {c.v[0], c.v[1], c.v[2], c.v[3]};
    cv = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bv, cv, 0, 0, 0);
    for (int j = 0; j < 4; ++j) c.v[j] = cv[j];
    return c;
}

__device__ __forceinline__ Frag<float, 16, 16, Accumulator> mma(const Frag<f16, 16, 32, MatrixA>& a,
                                                                const Frag<f16, 32, 16, MatrixB>& b,
                                                                Frag<float, 16, 16, Accumulator> c) {
    f16x8 av, bv;
#pragma unroll
    for (int j = 0; j < 8; ++j) { av[j] = a.v[j]; bv[j] = b.v[j]; }
    f32x4 cv = {c.v[0], c.v[1], c.v[2], c.v[3]};
    cv = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, cv, 0, 0, 0);
    for (int j = 0; j < 4; ++j) c.v[j] = cv[j];
    return c;
}

__device__ __forceinline__ Frag<float, 16, 16, Accumulator> mma(const Frag<bf16, 16, 32, MatrixA>& a,
                                                                const Frag<bf16, 32, 16, MatrixB>& b,
                                                                Frag<float, 16, 16, Accumulator> c) {
    bf16x8 av, bv;
#pragma unroll
    for (int j = 0; j < 8; ++j) { av[j] = a.v[j]; bv[j] = b.v[j]; }
    f32x4 cv = {c.v[0], c.v[1], c.v[2], c.v[3]};
    cv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, cv, 0, 0, 0);
    for (int j = 0; j < 4; ++j) c.v[j] = cv[j];
    return c;
}

__device__ __forceinline__ Frag<float, 32, 32, Accumulator> mma(const Frag<f16, 32, 16, MatrixA>& a,
                                                                const Frag<f16, 16, 32, MatrixB>& b,
                                                                Frag<float, 32, 32, Accumulator> c) {
    f16x8 av, bv;
#pragma unroll
    for (int j = 0; j < 8; ++j) { av[j] = a.v[j]; bv[j] = b.v[j]; }
    f32x16 cv;
#pragma unroll
    for (int j = 0; j < 16; ++j) cv[j] = c.v[j];
    cv = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, cv, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 16; ++j) c.v[j] = cv[j];
    return c;
}

__device__ __forceinline__ Frag<float, 32, 32, Accumulator> mma(const Frag<bf16, 32, 16, MatrixA>& a,
                                                                const Frag<bf16, 16, 32, MatrixB>& b,
                                                                Frag<float, 32, 32, Accumulator> c) {
    bf16x8 av, bv;
#pragma unroll
    for (int j = 0; j < 8; ++j) { av[j] = a.v[j]; bv[j] = b.v[j]; }
    f32x16 cv;
#pragma unroll
    for (int j = 0; j < 16; ++j) cv[j] = c.v[j];
    cv = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, cv, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 16; ++j) c.v[j] = cv[j];
    return c;
}

// int8 x int8 -> int32, signed operands, 16x16x16: the 16x16x32 instruction with
// the upper half of each lane's k slots zero.
__device__ __forceinline__ Frag<int32_t, 16, 16, Accumulator> mma(const Frag<int8_t, 16, 16, MatrixA>& a,
                                                                  const Frag<int8_t, 16, 16, MatrixB>& b,
                                                                  Frag<int32_t, 16, 16, Accumulator> c) {
    uint32_t alo = 0, blo = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        alo |= (uint32_t)(uint8_t)a.v[j] << (8 * j);
        blo |= (uint32_t)(uint8_t)b.v[j] << (8 * j);
    }
    long av = (long)(uint64_t)alo, bv = (long)(uint64_t)blo;
    i32x4 cv = {c.v[0], c.v[1], c.v[2], c.v[3]};
    cv = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, cv, 0, 0, 0);
    for (int j = 0; j < 4; ++j) c.v[j] = cv[j];
    return c;
}

__device__ __forceinline__ Frag<int32_t, 16, 16, Accumulator> mma(const Frag<int8_t, 16, 64, MatrixA>& a,
                                                                  const Frag<int8_t, 64, 16, MatrixB>& b,
                                                                  Frag<int32_t, 16, 16, Accumulator> c) {
    i32x4 av, bv;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t x = 0, y = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x |= (uint32_t)(uint8_t)a.v[4 * w + j] << (8 * j);
            y |= (uint32_t)(uint8_t)b.v[4 * w + j] << (8 * j);
        }
        av[w] = (int)x;
        bv[w] = (int)y;
    }
    i32x4 cv = {c.v[0], c.v[1], c.v[2], c.v[3]};
    cv = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, cv, 0, 0, 0);
    for (int j = 0; j < 4; ++j) c.v[j] = cv[j];
    return c;
}

// dot4x8 (src/vocabulary/vocabulary.jl:31-35): v_dot4_i32_i8
__device__ __forceinline__ int32_t dot4x8(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, 0, false);
}

}  // namespace lava
