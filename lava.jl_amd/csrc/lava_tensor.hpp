// lava_tensor.hpp -- tensor addressing over the cooperative-matrix fragments.
//
// Lava's TensorLayout / TensorView vocabulary (src/vocabulary/tensor.jl:1-115,
// lowered in src/device/tensor_intrinsics.jl): a layout describes an array in
// memory -- extents and element strides per dimension, innermost last -- plus a
// slice (the block one workgroup or one matrix reads) and a clamp mode for
// elements of the slice that fall outside the tensor.  A matrix is loaded from and
// stored to a layout directly, with no shared-memory staging.  On CDNA4 there is no
// tensor-addressing unit: each lane computes the addresses of the components it
// holds (the fragment's lane map) and bounds-checks them itself.
//
// Semantics (tensor.jl:44-51, tensor_intrinsics.jl `lava_tensor_load`/`_store`):
//  * the matrix's (row, col) is the slice's coordinate in its last two dimensions
//    -- (col, row) through a transposing view, PERM = (1, 0); the outer dimensions
//    of a rank-3/4 slice are selected by its offsets (their sizes are 1);
//  * load: an element outside the slice's sizes keeps the object matrix's value; an
//    element inside the slice but outside the tensor reads the clamp constant
//    (TENSOR_CLAMP_CONSTANT, default zero), the nearest element inside
//    (TENSOR_CLAMP_TO_EDGE), or keeps the object's value (TENSOR_CLAMP_UNDEFINED:
//    "elements a clamping layout leaves out keep m's values", tensor.jl:98-104);
//  * store: only elements inside both the slice and the tensor are written;
//  * the clamp value is given as bits, those of the value in the matrix's component
//    type zero-extended (tensor_clampbits, tensor.jl:83-85).
#pragma once
#include <type_traits>

#include "lava_coopmat.hpp"

namespace lava {

enum TensorClamp : uint32_t { ClampUndefined = 0u, ClampConstant = 1u, ClampToEdge = 2u };

template <int DIM>
struct TensorLayout {
    static_assert(DIM >= 2 && DIM <= 4, "tensor layouts of rank 2 to 4");
    int32_t dim[DIM];      // extents, outermost first
    int32_t stride[DIM];   // element strides, same order
    int32_t off[DIM];      // slice origin (0-based, may be negative)
    int32_t size[DIM];     // slice extent
    uint32_t clamp;        // TensorClamp
    uint32_t clampbits;    // the clamp constant's bits in the component type
};

// tensor_layout(Val(DIM), Val(CLAMP)) + tensor_setdim: a packed tensor, sliced whole.
template <int DIM>
__host__ __device__ inline TensorLayout<DIM> tensor_layout(uint32_t clamp, const int32_t (&dims)[DIM]) {
    TensorLayout<DIM> l;
    int32_t s = 1;
    for (int d = DIM - 1; d >= 0; --d) {
        l.dim[d] = dims[d];
        l.stride[d] = s;
        s *= dims[d];
        l.off[d] = 0;
        l.size[d] = dims[d];
    }
    l.clamp = clamp;
    l.clampbits = 0u;
    return l;
}

// tensor_setstride: element strides, innermost last.
template <int DIM>
__host__ __device__ inline TensorLayout<DIM> tensor_setstride(TensorLayout<DIM> l, const int32_t (&strides)[DIM]) {
    for (int d = 0; d < DIM; ++d) l.stride[d] = strides[d];
    return l;
}

// tensor_setclampvalue: bits of the constant a TENSOR_CLAMP_CONSTANT load reads outside.
template <int DIM>
__host__ __device__ inline TensorLayout<DIM> tensor_setclampvalue(TensorLayout<DIM> l, uint32_t bits) {
    l.clampbits = bits;
    return l;
}

// tensor_slice: the block at `offs` (0-based, per dimension) of extent `sizes`.
template <int DIM>
__host__ __device__ inline TensorLayout<DIM> tensor_slice(TensorLayout<DIM> l, const int32_t (&offs)[DIM],
                                                          const int32_t (&sizes)[DIM]) {
    for (int d = 0; d < DIM; ++d) {
        l.off[d] = offs[d];
        l.size[d] = sizes[d];
    }
    return l;
}

// The component a clamp constant stands for: its bits in T, zero-extended.
template <typename T>
__device__ __forceinline__ T clamp_value(uint32_t bits) {
    if constexpr (sizeof(T) == 2) {
        const uint16_t u = (uint16_t)bits;
        return __builtin_bit_cast(T, u);
    } else if constexpr (std::is_same<T, float>::value) {
        return __builtin_bit_cast(float, bits);
    } else {
        return (T)(int32_t)bits;   // integer components: Int32(x)
    }
}

// Element offset of the slice's outer (rank > 2) block; `inside` says whether that
// block lies inside the tensor (TO_EDGE: clamped into it).
template <int DIM>
__device__ __forceinline__ int64_t tensor_outer(const TensorLayout<DIM>& l, bool& inside) {
    int64_t o = 0;
    inside = true;
#pragma unroll
    for (int d = 0; d < DIM - 2; ++d) {
        int t = l.off[d];
        if (l.clamp == ClampToEdge && l.dim[d] > 0) t = t < 0 ? 0 : (t >= l.dim[d] ? l.dim[d] - 1 : t);
        inside = inside && t >= 0 && t < l.dim[d];
        o += (int64_t)t * l.stride[d];
    }
    return o;
}

// Element (i0, i1) of the slice's last two dimensions.  Returns false when it lies
// outside the slice (the caller keeps / skips it); otherwise `*idx` is its element
// offset and `*in` says whether it lies inside the tensor (TO_EDGE: clamped to it).
template <int DIM>
__device__ __forceinline__ bool tensor_elem(const TensorLayout<DIM>& l, int64_t outer, bool outer_in, int i0, int i1,
                                            int64_t* idx, bool* in) {
    constexpr int d0 = DIM - 2, d1 = DIM - 1;
    if (i0 >= l.size[d0] || i1 >= l.size[d1]) return false;
    int t0 = l.off[d0] + i0, t1 = l.off[d1] + i1;
    bool inside = outer_in && t0 >= 0 && t0 < l.dim[d0] && t1 >= 0 && t1 < l.dim[d1];
    if (!inside && l.clamp == ClampToEdge && outer_in && l.dim[d0] > 0 && l.dim[d1] > 0) {
        t0 = t0 < 0 ? 0 : (t0 >= l.dim[d0] ? l.dim[d0] - 1 : t0);
        t1 = t1 < 0 ? 0 : (t1 >= l.dim[d1] ? l.dim[d1] - 1 : t1);
        inside = true;
    }
    *idx = outer + (int64_t)t0 * l.stride[d0] + (int64_t)t1 * l.stride[d1];
    *in = inside;
    return true;
}

// tensor_load(m, address, layout[, view]): `m` is the object whose components the
// elements outside the slice keep.  TRANS = the (1, 0) view.
template <bool TRANS = false, typename T, int R, int C, Use U, int DIM>
__device__ __forceinline__ Frag<T, R, C, U> tensor_load(Frag<T, R, C, U> m, const T* base,
                                                        const TensorLayout<DIM>& l) {
    using L = Layout<R, C, U>;
    const int lane = lane_id();
    bool outer_in;
    const int64_t outer = tensor_outer(l, outer_in);
    const T cval = clamp_value<T>(l.clampbits);
#pragma unroll
    for (int j = 0; j < L::len; ++j) {
        const int r = L::row(lane, j), c = L::col(lane, j);
        int64_t idx;
        bool in;
        if (!tensor_elem(l, outer, outer_in, TRANS ? c : r, TRANS ? r : c, &idx, &in)) continue;
        if (in)
            m.v[j] = base[idx];
        else if (l.clamp != ClampUndefined)
            m.v[j] = cval;
    }
    return m;
}

// tensor_store(m, address, layout[, view]): the clamping store.
template <bool TRANS = false, typename S, typename T, int R, int C, Use U, int DIM>
__device__ __forceinline__ void tensor_store(const Frag<T, R, C, U>& m, S* base, const TensorLayout<DIM>& l) {
    using L = Layout<R, C, U>;
    const int lane = lane_id();
    bool outer_in;
    const int64_t outer = tensor_outer(l, outer_in);
    TensorLayout<DIM> ls = l;
    ls.clamp = ClampConstant;   // a store never clamps to the edge: outside is dropped
#pragma unroll
    for (int j = 0; j < L::len; ++j) {
        const int r = L::row(lane, j), c = L::col(lane, j);
        int64_t idx;
        bool in;
        if (!tensor_elem(ls, outer, outer_in, TRANS ? c : r, TRANS ? r : c, &idx, &in) || !in) continue;
        base[idx] = (S)m.v[j];
    }
}

}  // namespace lava
