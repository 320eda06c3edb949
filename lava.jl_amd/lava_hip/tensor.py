"""Tensor addressing: the host half of Lava's TensorLayout / TensorView vocabulary.

Mirrors src/vocabulary/tensor.jl (KernelInterface's tensor operations): a layout is
built with `tensor_layout(rank, clamp)`, given extents with `tensor_setdim` (which
also makes it packed and slices it whole), strides with `tensor_setstride`, a clamp
constant with `tensor_setclampvalue(layout, tensor_clampbits(x, T))`, and cut to one
block with `tensor_slice` (0-based offsets, sizes); `tensor_view(rank, (1, 0))` is
the transposing view.  Layouts are immutable values, as in Lava (each call returns a
new one).  The device side of the same vocabulary is lava_tensor.hpp; the entry
points here load or store one fragment through a layout, multiply two fragments
loaded through layouts, and run the coopmat2 GEMM.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, replace
from typing import Optional

import numpy as np

from . import _lib
from .device import HIPDeviceArray

TENSOR_CLAMP_UNDEFINED = 0
TENSOR_CLAMP_CONSTANT = 1
TENSOR_CLAMP_TO_EDGE = 2

# fragment shapes of the tile entry points: name -> (code, rows, cols)
TILES = {"A16x16": (0, 16, 16), "B16x16": (1, 16, 16), "acc16x16": (2, 16, 16), "acc32x32": (3, 32, 32),
         "A32x16": (4, 32, 16), "B16x32": (5, 16, 32)}


class CTensorLayout(C.Structure):
    """`lava_hip_tensor_layout` of include/lava_hip.h."""
    _fields_ = [("rank", C.c_int32), ("clamp", C.c_uint32), ("clampbits", C.c_uint32),
                ("dim", C.c_int32 * 4), ("stride", C.c_int32 * 4), ("off", C.c_int32 * 4),
                ("size", C.c_int32 * 4)]


@dataclass(frozen=True)
class TensorLayout:
    """TensorLayout{DIM,CLAMP} (tensor.jl:1-30): extents and strides outermost first,
    innermost last; the slice (offsets, sizes); the clamp constant's bits."""
    rank: int
    clamp: int
    dims: tuple = ()
    strides: tuple = ()
    offsets: tuple = ()
    sizes: tuple = ()
    clampbits: int = 0

    def to_c(self) -> CTensorLayout:
        c = CTensorLayout()
        c.rank = self.rank
        c.clamp = self.clamp
        c.clampbits = self.clampbits & 0xFFFFFFFF
        for i in range(self.rank):
            c.dim[i] = self.dims[i]
            c.stride[i] = self.strides[i]
            c.off[i] = self.offsets[i]
            c.size[i] = self.sizes[i]
        return c

    def as_dict(self) -> dict:
        return {"rank": self.rank, "clamp": self.clamp, "dim": list(self.dims), "stride": list(self.strides),
                "off": list(self.offsets), "size": list(self.sizes), "clampbits": self.clampbits}


@dataclass(frozen=True)
class TensorView:
    """TensorView{DIM,PERM} (tensor.jl:32-42): a dimension permutation applied at a load."""
    rank: int
    perm: tuple


def _tuple(x, rank: int, what: str) -> tuple:
    t = tuple(int(v) for v in x)
    if len(t) != rank:
        raise ValueError(f"{what}: {len(t)} values for a rank-{rank} layout")
    if any(v < -2 ** 31 or v >= 2 ** 31 for v in t):
        raise ValueError(f"{what}: values are 32-bit in a tensor layout")
    return t


def tensor_layout(rank: int, clamp: int = TENSOR_CLAMP_UNDEFINED) -> TensorLayout:
    """A fresh layout (tensor.jl:52-59); extents come from tensor_setdim."""
    if rank not in (2, 3, 4):
        raise ValueError("tensor layouts of rank 2, 3 or 4")
    if clamp not in (TENSOR_CLAMP_UNDEFINED, TENSOR_CLAMP_CONSTANT, TENSOR_CLAMP_TO_EDGE):
        raise ValueError(f"unknown clamp mode {clamp}")
    z = (0,) * rank
    return TensorLayout(rank, clamp, z, z, z, z, 0)


def tensor_setdim(l: TensorLayout, dims) -> TensorLayout:
    """The extent per dimension (tensor.jl:61-62): the layout becomes packed and sliced whole."""
    d = _tuple(dims, l.rank, "tensor_setdim")
    if any(v < 0 for v in d):
        raise ValueError("tensor_setdim: negative extent")
    strides, s = [0] * l.rank, 1
    for i in range(l.rank - 1, -1, -1):
        strides[i] = s
        s *= d[i]
    return replace(l, dims=d, strides=tuple(strides), offsets=(0,) * l.rank, sizes=d)


def tensor_setstride(l: TensorLayout, strides) -> TensorLayout:
    """The stride per dimension in elements, innermost last (tensor.jl:64-65)."""
    return replace(l, strides=_tuple(strides, l.rank, "tensor_setstride"))


def tensor_setclampvalue(l: TensorLayout, bits: int) -> TensorLayout:
    """What a TENSOR_CLAMP_CONSTANT load reads outside the tensor, as tensor_clampbits gives it (tensor.jl:67-73)."""
    return replace(l, clampbits=int(bits))


def tensor_clampbits(x, dtype: str) -> int:
    """The bits of x in the component type, zero-extended (tensor.jl:83-85)."""
    if dtype == "f16":
        return int(np.array([x], dtype=np.float16).view(np.uint16)[0])
    if dtype == "f32":
        return int(np.array([x], dtype=np.float32).view(np.int32)[0])
    if dtype in ("i8", "u8", "i32", "u32"):
        return int(x)
    raise ValueError(f"no clamp bits for {dtype}")


def tensor_slice(l: TensorLayout, offsets, sizes) -> TensorLayout:
    """The block at 0-based `offsets` of extent `sizes` (tensor.jl:87-93)."""
    sz = _tuple(sizes, l.rank, "tensor_slice sizes")
    if any(v < 0 for v in sz):
        raise ValueError("tensor_slice: negative size")
    return replace(l, offsets=_tuple(offsets, l.rank, "tensor_slice offsets"), sizes=sz)


def tensor_view(rank: int, perm) -> TensorView:
    """A dimension permutation (tensor.jl:95-96).  The device path implements the identity
    and the swap of the last two dimensions (the transpose)."""
    p = tuple(int(v) for v in perm)
    if sorted(p) != list(range(rank)):
        raise ValueError(f"{p} is not a permutation of {rank} dimensions")
    return TensorView(rank, p)


def _transpose_flag(view: Optional[TensorView], rank: int) -> int:
    if view is None:
        return 0
    if view.rank != rank:
        raise ValueError(f"a rank-{view.rank} view on a rank-{rank} layout")
    ident = tuple(range(rank))
    swap = ident[:-2] + (rank - 1, rank - 2)
    if view.perm == ident:
        return 0
    if view.perm == swap:
        return 1
    raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, f"view {view.perm}: only the identity and the transpose of the "
                                                 "last two dimensions")


def _tile(shape: str):
    if shape not in TILES:
        raise ValueError(f"tile shape must be one of {sorted(TILES)}")
    return TILES[shape]


def _check_tile_array(a: HIPDeviceArray, R: int, Cc: int, what: str):
    if a.dims != (R, Cc) or a.order != "C":
        raise ValueError(f"{what} must be a row-major {R} x {Cc} array, got {a.dims} order {a.order}")


def tensor_load_tile(out: HIPDeviceArray, src: HIPDeviceArray, layout: TensorLayout, obj: HIPDeviceArray,
                     shape: str, view: Optional[TensorView] = None, stream: Optional[int] = None) -> HIPDeviceArray:
    """out = tensor_load(obj, src, layout[, view]) for one fragment of `shape`
    (src/device/tensor_intrinsics.jl:258-320).  `src` holds the tensor the layout
    describes; `obj` and `out` are row-major R x C arrays of the same dtype."""
    code, R, Cc = _tile(shape)
    _check_tile_array(out, R, Cc, "out")
    _check_tile_array(obj, R, Cc, "object")
    if not (out.dtype == obj.dtype == src.dtype):
        raise ValueError("src, object and out must share a dtype")
    lc = layout.to_c()
    _lib.call("lava_hip_tensor_load_tile", out.code, code, src.ptr, C.byref(lc),
              _transpose_flag(view, layout.rank), obj.ptr, out.ptr, stream)
    return out


def tensor_store_tile(dst: HIPDeviceArray, inp: HIPDeviceArray, layout: TensorLayout, shape: str,
                      view: Optional[TensorView] = None, stream: Optional[int] = None) -> HIPDeviceArray:
    """tensor_store(m, dst, layout[, view]) of the fragment read from row-major `inp`: the
    clamping store (src/device/tensor_intrinsics.jl:329-402)."""
    code, R, Cc = _tile(shape)
    _check_tile_array(inp, R, Cc, "in")
    if inp.dtype != dst.dtype:
        raise ValueError("in and dst must share a dtype")
    lc = layout.to_c()
    _lib.call("lava_hip_tensor_store_tile", inp.code, code, inp.ptr, dst.ptr, C.byref(lc),
              _transpose_flag(view, layout.rank), stream)
    return dst


def tensor_muladd_16x16x16(D: HIPDeviceArray, A: HIPDeviceArray, layout_a: TensorLayout, B: HIPDeviceArray,
                           layout_b: TensorLayout, view_b: Optional[TensorView] = None,
                           stream: Optional[int] = None) -> HIPDeviceArray:
    """D (16 x 16 fp32, row-major) = A * B, both fp16 operands loaded through layouts."""
    _check_tile_array(D, 16, 16, "D")
    if D.dtype != "f32" or A.dtype != "f16" or B.dtype != "f16":
        raise ValueError("fp16 operands, fp32 D")
    la, lb = layout_a.to_c(), layout_b.to_c()
    _lib.call("lava_hip_tensor_muladd_16x16x16", A.ptr, C.byref(la), B.ptr, C.byref(lb),
              _transpose_flag(view_b, layout_b.rank), D.ptr, stream)
    return D


def gemm_cm2(Cm: HIPDeviceArray, A: HIPDeviceArray, B: HIPDeviceArray, transpose: bool = False,
             vocabulary: bool = False, stream: Optional[int] = None) -> HIPDeviceArray:
    """The coopmat2 GEMM (test/glsl/coopmat2_gemm_regs.comp:37-84): fp16 A (M x K) and B
    (K x N) row-major, fp32 accumulate, fp16 C (M x N) row-major -- or, transpose=True,
    C^T into an N x M row-major array through the transposing view.  Any M, N, K.
    vocabulary=True runs the shader's own form written with tensor_load / tensor_store
    instead of the 256 x 256 tile kernel."""
    if not (A.dtype == B.dtype == Cm.dtype == "f16"):
        raise ValueError("gemm_cm2 is fp16 in, fp16 out")
    if A.order != "C" or B.order != "C" or Cm.order != "C":
        raise ValueError("gemm_cm2 operands are row-major (order 'C')")
    M, K = A.dims
    K2, N = B.dims
    want = (N, M) if transpose else (M, N)
    if K2 != K or Cm.dims != want:
        raise ValueError(f"shape mismatch: A {A.dims}, B {B.dims}, C {Cm.dims} (want {want})")
    flags = (1 if transpose else 0) | (2 if vocabulary else 0)
    _lib.call("lava_hip_gemm_cm2_f16", A.ptr, B.ptr, Cm.ptr, M, N, K, max(K, 1), max(N, 1), max(Cm.dims[1], 1),
              flags, stream)
    return Cm
