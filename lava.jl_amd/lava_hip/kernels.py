"""The hot-path kernels, called destination-first as a Lava kernel launch is
(`gemm!(C, A, B)`, like README.md's `vadd!(c, a, b)`), over HIPDeviceArrays or raw
device addresses.

Every function forwards to one entry point of liblava_hip.so; argument errors
come back as InvalidArgument / Unsupported without touching the GPU.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence

from . import _lib
from .device import HIPDeviceArray

_GEMM_ENTRY = {("f16", "f32"): "lava_hip_gemm_f16_f32", ("bf16", "f32"): "lava_hip_gemm_bf16_f32",
               ("i8", "i32"): "lava_hip_gemm_i8_i32", ("u8", "u32"): "lava_hip_gemm_u8_u32"}


def _ld(a: HIPDeviceArray) -> int:
    """Leading dimension of a 2-D array in its own order."""
    if len(a.dims) != 2:
        raise ValueError(f"expected a matrix, got dims {a.dims}")
    return max(1, a.dims[0] if a.order == "F" else a.dims[1])


def gemm_raw(ab: str, acc: str, A: int, B: int, C_: int, M: int, N: int, K: int, lda: int, ldb: int, ldc: int,
             layout: int, stream: Optional[int] = None) -> None:
    """C = A * B on raw device addresses; layout bits: A/B/C row-major (1/2/4)."""
    try:
        name = _GEMM_ENTRY[(ab, acc)]
    except KeyError:
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, f"no GEMM for {ab} -> {acc}") from None
    _lib.call(name, A, B, C_, M, N, K, lda, ldb, ldc, layout, stream)


def gemm(C_: HIPDeviceArray, A: HIPDeviceArray, B: HIPDeviceArray, stream: Optional[int] = None) -> HIPDeviceArray:
    """`C = A * B` (muladd(a, b, zero(c)), src/vocabulary/coopmat.jl:196-203) with each
    operand's own storage order."""
    if A.dtype != B.dtype:
        raise ValueError(f"A is {A.dtype}, B is {B.dtype}")
    M, K = A.dims
    K2, N = B.dims
    if K2 != K or C_.dims != (M, N):
        raise ValueError(f"shape mismatch: A {A.dims}, B {B.dims}, C {C_.dims}")
    layout = (1 if A.order == "C" else 0) | (2 if B.order == "C" else 0) | (4 if C_.order == "C" else 0)
    gemm_raw(A.dtype, C_.dtype, A.ptr, B.ptr, C_.ptr, M, N, K, _ld(A), _ld(B), _ld(C_), layout, stream)
    return C_


_ACTS = {"none": _lib.ACT_NONE, "relu": _lib.ACT_RELU, "gelu_tanh": _lib.ACT_GELU_TANH,
         "gelu_erf": _lib.ACT_GELU_ERF}
_DCODE = {"f16": _lib.F16, "bf16": _lib.BF16, "f32": _lib.F32}


def gemm_ex_raw(ab: str, d: str, A: int, B: int, D: int, M: int, N: int, K: int, lda: int, ldb: int, ldd: int,
                layout: int, bias: int = 0, residual: int = 0, ldr: int = 0, act: str = "none",
                stream: Optional[int] = None) -> None:
    """D = act(A*B + (bias + residual)) narrowed to `d`, on raw device addresses."""
    if act not in _ACTS:
        raise ValueError(f"act must be one of {sorted(_ACTS)}")
    if ab not in ("f16", "bf16") or d not in _DCODE:
        raise _lib.Unsupported(_lib.ERR_UNSUPPORTED, f"no fused GEMM for {ab} -> {d}")
    _lib.call("lava_hip_gemm_ex", _DCODE[ab], _DCODE[d], A, B, D, M, N, K, lda, ldb, ldd, layout, bias or None,
              residual or None, ldr, _ACTS[act], stream)


def gemm_ex(D: HIPDeviceArray, A: HIPDeviceArray, B: HIPDeviceArray, bias: Optional[HIPDeviceArray] = None,
            residual: Optional[HIPDeviceArray] = None, act: str = "none",
            stream: Optional[int] = None) -> HIPDeviceArray:
    """`D = act(A*B + (bias + residual))` with D fp32, fp16 or bf16: the GEMM epilogue family
    fused into the store -- Lava's `accinit` (bias at stride 0, one value per row of D, plus
    the residual, src/device/coopmat_intrinsics.jl:435-464), an elementwise getcomp/setcomp
    epilogue (relu, gelu_tanh, gelu_erf) and the narrowing coopmat_convert (RNE)."""
    if A.dtype != B.dtype:
        raise ValueError(f"A is {A.dtype}, B is {B.dtype}")
    M, K = A.dims
    K2, N = B.dims
    if K2 != K or D.dims != (M, N):
        raise ValueError(f"shape mismatch: A {A.dims}, B {B.dims}, D {D.dims}")
    if bias is not None and (bias.dtype != "f32" or bias.size != M):
        raise ValueError("bias must be an f32 vector of length M (one value per row of D)")
    if residual is not None and (residual.dtype != "f32" or residual.dims != (M, N) or residual.order != D.order):
        raise ValueError("residual must be an f32 M x N array in D's order")
    layout = (1 if A.order == "C" else 0) | (2 if B.order == "C" else 0) | (4 if D.order == "C" else 0)
    gemm_ex_raw(A.dtype, D.dtype, A.ptr, B.ptr, D.ptr, M, N, K, _ld(A), _ld(B), _ld(D), layout,
                bias.ptr if bias is not None else 0, residual.ptr if residual is not None else 0,
                _ld(residual) if residual is not None else 0, act, stream)
    return D


def coopmat_gemm_tiles(C_: HIPDeviceArray, A: HIPDeviceArray, B: HIPDeviceArray,
                       stream: Optional[int] = None) -> HIPDeviceArray:
    """The 16x16x16 vocabulary-tile GEMM of docs/src/device.md:81-88 (fp16 -> fp32)."""
    if A.dtype != "f16" or B.dtype != "f16" or C_.dtype != "f32":
        raise ValueError(f"the tile GEMM is f16 x f16 -> f32 (got {A.dtype}, {B.dtype}, {C_.dtype})")
    M, K = A.dims
    K2, N = B.dims
    if K2 != K or C_.dims != (M, N):
        raise ValueError(f"shape mismatch: A {A.dims}, B {B.dims}, C {C_.dims}")
    layout = (1 if A.order == "C" else 0) | (2 if B.order == "C" else 0) | (4 if C_.order == "C" else 0)
    _lib.call("lava_hip_coopmat_gemm_f16_tiles", A.ptr, B.ptr, C_.ptr, M, N, K, _ld(A), _ld(B), _ld(C_), layout,
              stream)
    return C_


def _check_w8a16(Y: HIPDeviceArray, X: HIPDeviceArray, W: HIPDeviceArray, scale: HIPDeviceArray) -> None:
    if (X.dtype, W.dtype, scale.dtype, Y.dtype) != ("f16", "i8", "f16", "f32"):
        raise ValueError(f"W8A16 is f16 X, i8 W, f16 scale -> f32 Y (got {X.dtype}, {W.dtype}, {scale.dtype}, "
                         f"{Y.dtype})")
    if len(X.dims) != 2 or len(W.dims) != 2 or len(Y.dims) != 2:
        raise ValueError("X, W and Y must be 2-D")
    M, K = X.dims
    K2, N = W.dims
    if K2 != K or Y.dims != (M, N) or scale.size != N:
        raise ValueError(f"shape mismatch: X {X.dims}, W {W.dims}, scale {scale.dims}, Y {Y.dims}")


def w8a16(Y: HIPDeviceArray, X: HIPDeviceArray, W: HIPDeviceArray, scale: HIPDeviceArray,
          stream: Optional[int] = None) -> HIPDeviceArray:
    """Y = (X * float(W)) .* scale[col]: the per-element dequant epilogue
    (src/device/coopmat_intrinsics.jl:535-628)."""
    _check_w8a16(Y, X, W, scale)
    M, K = X.dims
    N = W.dims[1]
    layout = (1 if X.order == "C" else 0) | (2 if W.order == "C" else 0) | (4 if Y.order == "C" else 0)
    _lib.call("lava_hip_gemm_w8a16", X.ptr, W.ptr, scale.ptr, Y.ptr, M, N, K, _ld(X), _ld(W), _ld(Y), layout,
              stream)
    return Y


def w8a16_noalloc(Y: HIPDeviceArray, X: HIPDeviceArray, W: HIPDeviceArray, scale: HIPDeviceArray,
                  stream: Optional[int] = None) -> HIPDeviceArray:
    """`w8a16` through the entry point that allocates nothing: the split-K partials live in a
    fixed per-GPU device array (shared by every call on that GPU: overlapping calls race)."""
    _check_w8a16(Y, X, W, scale)
    M, K = X.dims
    N = W.dims[1]
    layout = (1 if X.order == "C" else 0) | (2 if W.order == "C" else 0) | (4 if Y.order == "C" else 0)
    _lib.call("lava_hip_gemm_w8a16_noalloc", X.ptr, W.ptr, scale.ptr, Y.ptr, M, N, K, _ld(X), _ld(W), _ld(Y), layout,
              stream)
    return Y


def w8a16_raw(X: int, W: int, scale: int, Y: int, M: int, N: int, K: int, ldx: int, ldw: int, ldy: int,
              layout: int = 7, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_gemm_w8a16", X, W, scale, Y, M, N, K, ldx, ldw, ldy, layout, stream)


def flash_attn_fwd_raw(Q: int, K: int, V: int, O: int, B: int, H: int, S: int, D: int,
                       strides: Sequence[int], ostrides: Optional[Sequence[int]] = None,
                       scale: Optional[float] = None, causal: bool = True, stream: Optional[int] = None) -> None:
    st = (C.c_int64 * 4)(*strides)
    ost = (C.c_int64 * 4)(*ostrides) if ostrides is not None else None
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    _lib.call("lava_hip_flash_attn_fwd_f16", Q, K, V, O, B, H, S, D, st, ost, sc, int(bool(causal)), stream)


def flash_attn_fwd(O: HIPDeviceArray, Q: HIPDeviceArray, K: HIPDeviceArray, V: HIPDeviceArray,
                   scale: Optional[float] = None, causal: bool = True, stream: Optional[int] = None) -> HIPDeviceArray:
    """O = softmax(Q K^T * scale + causal mask) V over (E, L, H, B) fp16 arrays, head
    dimension fastest (src/device/tensor_intrinsics.jl:279-281)."""
    for t in (Q, K, V, O):
        if t.dtype != "f16" or len(t.dims) != 4:
            raise ValueError("Q, K, V, O must be 4-D f16 arrays (E, L, H, B)")
    if not (Q.dims == K.dims == V.dims == O.dims):
        raise ValueError("Q, K, V, O must share dims (E, L, H, B)")
    if Q.order != "F" or K.order != Q.order or V.order != Q.order:
        raise ValueError("Q, K, V must be column-major (E fastest)")
    E, L, H, Bn = Q.dims
    flash_attn_fwd_raw(Q.ptr, K.ptr, V.ptr, O.ptr, Bn, H, L, E, Q.strides(), O.strides(), scale, causal, stream)
    return O


# ---- tile-level vocabulary -------------------------------------------------------
def coopmat_muladd_16x16x16(ab: str, acc: str, A: int, offA: int, strideA: int, B: int, offB: int, strideB: int,
                            Cp: int, offC: int, strideC: int, D: int, offD: int, strideD: int, layout: int = 0,
                            ntiles: int = 1, tile_step: int = 0, stream: Optional[int] = None) -> None:
    """`copyto!(D, offD, strideD, muladd(a, b, c))` over 1-based offsets and element
    strides; layout bits 0..3 mark A, B, C, D row-major."""
    codes = {"f16": _lib.F16, "f32": _lib.F32, "i8": _lib.I8, "i32": _lib.I32, "u8": _lib.U8, "u32": _lib.U32,
             "f64": _lib.F64}
    _lib.call("lava_hip_coopmat_muladd_16x16x16", codes[ab], codes[acc], A, offA, strideA, B, offB, strideB, Cp,
              offC, strideC, D, offD, strideD, layout, ntiles, tile_step, stream)


def coopmat_perelement_rowcol(inp: int, out: int, tile: int, ntiles: int, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_coopmat_perelement_rowcol", inp, out, tile, ntiles, stream)


def coopmat_perelement_pair(m: int, o: int, out: int, tile: int, ntiles: int, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_coopmat_perelement_pair", m, o, out, tile, ntiles, stream)


def coopmat_reduce(inp: int, out: int, tile: int, mask: int, combine: str, ntiles: int,
                   stream: Optional[int] = None) -> None:
    comb = {"add": _lib.COMBINE_ADD, "max": _lib.COMBINE_MAX, "min": _lib.COMBINE_MIN}[combine]
    _lib.call("lava_hip_coopmat_reduce", inp, out, tile, mask, comb, ntiles, stream)


def coopmat_reduce_into(inp: int, out: int, tile: int, dst_rows: int, dst_cols: int, mask: int, combine: str,
                        ntiles: int, stream: Optional[int] = None) -> None:
    """coopmat_reduce into a destination of another extent (Row, Column, RowAndColumn smeared
    into dst_rows x dst_cols), or the TwoByTwo block reduce into tile/2 x tile/2; column-major
    fp32 tiles, ntiles of each."""
    comb = {"add": _lib.COMBINE_ADD, "max": _lib.COMBINE_MAX, "min": _lib.COMBINE_MIN}[combine]
    _lib.call("lava_hip_coopmat_reduce_into", inp, out, tile, dst_rows, dst_cols, mask, comb, ntiles, stream)


def coopmat_convert(inp: int, out: int, out_dtype: str, n: int, stream: Optional[int] = None) -> None:
    code = {"f16": _lib.F16, "bf16": _lib.BF16}[out_dtype]
    _lib.call("lava_hip_coopmat_convert", inp, out, code, n, stream)


_USES = {"MatrixA": _lib.USE_MATRIX_A, "MatrixB": _lib.USE_MATRIX_B, "Accumulator": _lib.USE_ACCUMULATOR}


def coopmat_convert_use(inp: int, out: int, out_dtype: str, tile: int, use: str, ntiles: int,
                        stream: Optional[int] = None) -> None:
    """convert(CoopMatrix{out_dtype,tile,tile,use}, m) of fp32 Accumulator tiles: narrowing
    (RNE) and a change of use (coopmat_intrinsics.jl:222-247), stored through the new use's
    lane map."""
    code = {"f16": _lib.F16, "bf16": _lib.BF16}[out_dtype]
    _lib.call("lava_hip_coopmat_convert_use", inp, out, code, tile, _USES[use], ntiles, stream)


def coopmat_convert_use_muladd(P: int, V: int, D: int, ntiles: int, stream: Optional[int] = None) -> None:
    """D = convert(MatrixA f16, P) * V on 16x16x16 tiles (attention's P_A step)."""
    _lib.call("lava_hip_coopmat_convert_use_muladd_16x16x16", P, V, D, ntiles, stream)


def coopmat_elementwise(op: str, tile: int, A: int, strideA: int, B: int, strideB: int, D: int, strideD: int,
                        layout: int = 0, ntiles: int = 1, tile_step: int = 0, stream: Optional[int] = None) -> None:
    """D = coopmat_mul(a, b) or coopmat_add(a, b); a stride of 0 loads a broadcast factor
    matrix (coopmat_intrinsics.jl:402-464).  layout bits 0..2: A, B, D row-major."""
    code = {"mul": _lib.ELEMENTWISE_MUL, "add": _lib.ELEMENTWISE_ADD}[op]
    _lib.call("lava_hip_coopmat_elementwise", code, tile, A, strideA, B, strideB, D, strideD, layout, ntiles,
              tile_step, stream)


def coopmat_accinit_muladd(A: int, B: int, bias: int, residual: int, ldr: int, D: int, ldd: int, ntiles: int = 1,
                           stream: Optional[int] = None) -> None:
    """D = muladd(a, b, add(bias at stride 0, residual)) on 16x16x16 tiles (`accinit`)."""
    _lib.call("lava_hip_coopmat_accinit_muladd_16x16x16", A, B, bias, residual, ldr, D, ldd, ntiles, stream)


def coopmat_foreach_act(inp: int, out: int, tile: int, act: str, ntiles: int, length_out: int,
                        stream: Optional[int] = None) -> None:
    """for i in 0:length-1: setcomp(m, i, act(getcomp(m, i))) (coopmat_intrinsics.jl:322-400)."""
    if act not in _ACTS:
        raise ValueError(f"act must be one of {sorted(_ACTS)}")
    _lib.call("lava_hip_coopmat_foreach_act", inp, out, tile, _ACTS[act], ntiles, length_out, stream)


def coopmat_length(dtype: str, rows: int, cols: int, use: str) -> int:
    """coopmat_length(CoopMatrix{dtype,rows,cols,use}): components per lane."""
    codes = {"f16": _lib.F16, "bf16": _lib.BF16, "f32": _lib.F32, "i8": _lib.I8, "i32": _lib.I32}
    n = C.c_int32()
    _lib.call("lava_hip_coopmat_length", codes[dtype], rows, cols, _USES[use], C.byref(n))
    return int(n.value)


def coopmat_perelement_scale(inp: int, out: int, tile: int, by_row: bool, factors: int, base: int, ntiles: int,
                             stream: Optional[int] = None) -> None:
    """coopmat_perelement(f, m, ptr, base): e * s[base + col] (fp16 s, the W8A16 dequant) or
    e * cs[base + row] (fp32 cs, the attention rescale) (coopmat_intrinsics.jl:569-628)."""
    _lib.call("lava_hip_coopmat_perelement_scale", inp, out, tile, int(bool(by_row)), factors, base, ntiles, stream)


def coopmat_workgroup_gemm(C_: HIPDeviceArray, A: HIPDeviceArray, B: HIPDeviceArray, invocations: int,
                           stream: Optional[int] = None) -> HIPDeviceArray:
    """C = A * B as one workgroup-scope matrix held by a workgroup of `invocations` lanes;
    (M, N, K) must be multiples of wggranularity(caps(), invocations)."""
    if A.dtype != "f16" or B.dtype != "f16" or C_.dtype != "f32":
        raise ValueError("workgroup GEMM is fp16 x fp16 -> fp32")
    M, K = A.dims
    K2, N = B.dims
    if K2 != K or C_.dims != (M, N):
        raise ValueError(f"shape mismatch: A {A.dims}, B {B.dims}, C {C_.dims}")
    layout = (1 if A.order == "C" else 0) | (2 if B.order == "C" else 0) | (4 if C_.order == "C" else 0)
    _lib.call("lava_hip_coopmat_workgroup_gemm_f16", invocations, A.ptr, B.ptr, C_.ptr, M, N, K, _ld(A), _ld(B),
              _ld(C_), layout, stream)
    return C_


def dot4x8(a: int, b: int, y: int, n: int, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_dot4x8", a, b, y, n, stream)


# ---- seeded inputs on the device ------------------------------------------------------
def fill_uniform(dst: HIPDeviceArray, seed: int, a: float, b: float, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_fill_uniform", dst.ptr, dst.code, dst.size, seed, a, b, stream)


def fill_normal(dst: HIPDeviceArray, seed: int, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_fill_normal", dst.ptr, dst.code, dst.size, seed, stream)


def fill_i8(dst: HIPDeviceArray, seed: int, symmetric: bool = False, stream: Optional[int] = None) -> None:
    _lib.call("lava_hip_fill_i8", dst.ptr, dst.size, seed, int(bool(symmetric)), stream)
