"""CPU oracle for Lava.jl's cooperative-matrix path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module.  It is the checker, never the thing measured or shipped; the
product (liblava_hip.so and the lava_hip package) never imports it.

Each function names the reference definition it restates (paths relative to the
Lava.jl tree); the arithmetic is in oracle/lava_oracle.c (fp64 / exact integer)
or, for the tile-level definitions, plain numpy here.

Pinning (see tests/test_oracle.py): every function below is checked against an
independent source -- numpy/torch library routines (matmul, float16/bfloat16
casts, softmax), closed forms (identity, constant, one-hot inputs), brute force
on tiny inputs, or the reference's own known-answer definitions.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import math

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liblava_oracle.so"

F16, BF16, F32, I8, U8, I32 = 0, 1, 2, 3, 4, 5
_CODES = {"f16": F16, "bf16": BF16, "f32": F32, "i8": I8, "u8": U8, "i32": I32}

_lib = None


def build() -> Path:
    """Compile liblava_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liblava_oracle.so"], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        vp, i64, u64, u32 = C.c_void_p, C.c_int64, C.c_uint64, C.c_uint32
        L.oracle_rng_u64.restype = u64
        L.oracle_rng_u64.argtypes = [u64, u64]
        L.oracle_f32_to_f16.restype = C.c_uint16
        L.oracle_f32_to_f16.argtypes = [C.c_float]
        L.oracle_f32_to_bf16.restype = C.c_uint16
        L.oracle_f32_to_bf16.argtypes = [C.c_float]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_fill_uniform.argtypes = [vp, C.c_int, i64, u64, C.c_double, C.c_double]
        L.oracle_fill_normal.argtypes = [vp, C.c_int, i64, u64]
        L.oracle_fill_i8.argtypes = [vp, i64, u64, C.c_int]
        L.oracle_gemm_rows.argtypes = [vp, C.c_int, vp, C.c_int, i64, i64, i64, i64, i64, u32, vp, i64, vp]
        L.oracle_gemm_f32acc.argtypes = [vp, C.c_int, vp, C.c_int, i64, i64, i64, i64, u32, i64, vp]
        L.oracle_gemm_i8_rows.argtypes = [vp, vp, i64, i64, i64, i64, u32, vp, i64, vp]
        L.oracle_gemm_u8_rows.argtypes = [vp, vp, i64, i64, i64, i64, u32, vp, i64, vp]
        L.oracle_w8a16_rows.argtypes = [vp, vp, vp, i64, i64, i64, i64, vp, i64, vp]
        L.oracle_attn_rows.argtypes = [vp, vp, vp, i64, i64, vp, C.c_double, C.c_int, i64, i64, vp, i64, vp]
        L.oracle_dot4x8.restype = C.c_int32
        L.oracle_dot4x8.argtypes = [C.c_uint32, C.c_uint32]
        L.oracle_dot4x8_array.argtypes = [vp, vp, vp, i64]
        L.oracle_f32_to_f16_array.argtypes = [vp, vp, i64]
        L.oracle_f32_to_bf16_array.argtypes = [vp, vp, i64]
        L.oracle_num_threads.restype = C.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- generator -------------------------------------------------------------------
def rng_u64(seed: int, i: int) -> int:
    return int(lib().oracle_rng_u64(seed, i))


def fill_uniform(n: int, dtype: str, seed: int, a: float, b: float) -> np.ndarray:
    """f16 -> float16 array; bf16 -> uint16 bit patterns; f32 -> float32."""
    out = np.empty(n, dtype={"f16": np.float16, "bf16": np.uint16, "f32": np.float32}[dtype])
    lib().oracle_fill_uniform(_p(out), _CODES[dtype], n, seed, a, b)
    return out


def fill_normal(n: int, dtype: str, seed: int) -> np.ndarray:
    out = np.empty(n, dtype={"f16": np.float16, "bf16": np.uint16, "f32": np.float32}[dtype])
    lib().oracle_fill_normal(_p(out), _CODES[dtype], n, seed)
    return out


def fill_i8(n: int, seed: int, symmetric: bool = False) -> np.ndarray:
    out = np.empty(n, dtype=np.int8)
    lib().oracle_fill_i8(_p(out), n, seed, int(symmetric))
    return out


# ---- conversions ------------------------------------------------------------------------
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def decode(a: np.ndarray, dtype: str) -> np.ndarray:
    """Exact float64 values of an f16/bf16/f32 array."""
    if dtype == "bf16":
        return bf16_bits_to_f32(a).astype(np.float64)
    return np.asarray(a).astype(np.float64)


# ---- GEMM -------------------------------------------------------------------------------------
def gemm_rows(A: np.ndarray, adt: str, B: np.ndarray, bdt: str, M: int, N: int, K: int, lda: int, ldb: int,
              layout: int, rows) -> np.ndarray:
    """Rows `rows` of C = A*B in fp64; A and B are flat storage arrays addressed by
    layout (bit0 A row-major, bit1 B row-major)."""
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((rows.size, N), dtype=np.float64)
    A = np.ascontiguousarray(A)
    B = np.ascontiguousarray(B)
    lib().oracle_gemm_rows(_p(A), _CODES[adt], _p(B), _CODES[bdt], M, N, K, lda, ldb, layout, _p(rows), rows.size,
                           _p(out))
    return out


def gemm_f32acc(A: np.ndarray, adt: str, B: np.ndarray, bdt: str, N: int, K: int, lda: int, ldb: int, layout: int,
                nrows: int) -> np.ndarray:
    """The CPU baseline: rows [0, nrows) of A*B accumulated in fp32, all host threads."""
    out = np.empty((nrows, N), dtype=np.float32)
    A = np.ascontiguousarray(A)
    B = np.ascontiguousarray(B)
    lib().oracle_gemm_f32acc(_p(A), _CODES[adt], _p(B), _CODES[bdt], N, K, lda, ldb, layout, nrows, _p(out))
    return out


def gemm_i8_rows(A: np.ndarray, B: np.ndarray, N: int, K: int, lda: int, ldb: int, layout: int, rows) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((rows.size, N), dtype=np.int32)
    lib().oracle_gemm_i8_rows(_p(np.ascontiguousarray(A, dtype=np.int8)), _p(np.ascontiguousarray(B, dtype=np.int8)),
                              N, K, lda, ldb, layout, _p(rows), rows.size, _p(out))
    return out


def gemm_u8_rows(A: np.ndarray, B: np.ndarray, N: int, K: int, lda: int, ldb: int, layout: int, rows) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((rows.size, N), dtype=np.uint32)
    lib().oracle_gemm_u8_rows(_p(np.ascontiguousarray(A, dtype=np.uint8)),
                              _p(np.ascontiguousarray(B, dtype=np.uint8)), N, K, lda, ldb, layout, _p(rows),
                              rows.size, _p(out))
    return out


def w8a16_rows(X: np.ndarray, W: np.ndarray, s: np.ndarray, N: int, K: int, ldx: int, ldw: int, rows) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.empty((rows.size, N), dtype=np.float64)
    Xb = np.ascontiguousarray(X, dtype=np.float16).view(np.uint16)
    sb = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    lib().oracle_w8a16_rows(_p(Xb), _p(np.ascontiguousarray(W, dtype=np.int8)), _p(sb), N, K, ldx, ldw, _p(rows),
                            rows.size, _p(out))
    return out


# ---- attention ------------------------------------------------------------------------------------
def attn_rows(Q: np.ndarray, K: np.ndarray, V: np.ndarray, S: int, D: int, strides, scale: float, causal: bool,
              b: int, h: int, qrows) -> np.ndarray:
    """softmax(q K^T * scale + mask) V for query rows `qrows` of head (b, h), fp64.
    Q/K/V are flat fp16 storage with element (e,l,h,b) at dot((e,l,h,b), strides)."""
    qrows = np.ascontiguousarray(qrows, dtype=np.int64)
    st = np.ascontiguousarray(strides, dtype=np.int64)
    out = np.empty((qrows.size, D), dtype=np.float64)
    Qb = np.ascontiguousarray(Q, dtype=np.float16).view(np.uint16)
    Kb = np.ascontiguousarray(K, dtype=np.float16).view(np.uint16)
    Vb = np.ascontiguousarray(V, dtype=np.float16).view(np.uint16)
    lib().oracle_attn_rows(_p(Qb), _p(Kb), _p(Vb), S, D, _p(st), scale, int(causal), b, h, _p(qrows), qrows.size,
                           _p(out))
    return out


# ---- scalar / tile vocabulary -----------------------------------------------------------------------
def dot4x8(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint32)
    b = np.ascontiguousarray(b, dtype=np.uint32)
    out = np.empty(a.shape, dtype=np.int32)
    lib().oracle_dot4x8_array(_p(a), _p(b), _p(out), a.size)
    return out


def perelement_rowcol(m: np.ndarray) -> np.ndarray:
    """f(row, col, e) = e * (row + 1) + col, row/col 0-based
    (test/spirv/test_coopmat_perelement_inline.jl:20), in fp32."""
    r = np.arange(m.shape[0], dtype=np.float32)[:, None]
    c = np.arange(m.shape[1], dtype=np.float32)[None, :]
    return (m.astype(np.float32) * (r + np.float32(1)) + c).astype(np.float32)


def perelement_pair(m: np.ndarray, o: np.ndarray) -> np.ndarray:
    """f(row, col, x, y) = max(x, y) + row - col over corresponding elements
    (src/device/coopmat_intrinsics.jl:630-678), fp32."""
    r = np.arange(m.shape[0], dtype=np.float32)[:, None]
    c = np.arange(m.shape[1], dtype=np.float32)[None, :]
    return ((np.maximum(m, o).astype(np.float32) + r) - c).astype(np.float32)


def reduce_smear(m: np.ndarray, mask: int, combine: str) -> np.ndarray:
    """coopmat_reduce: combine along rows (mask 1), columns (2) or both (3); the
    result has m's shape with the value repeated (src/device/coopmat_intrinsics.jl:685-755)."""
    f = {"add": np.sum, "max": np.max, "min": np.min}[combine]
    x = m.astype(np.float64)
    if mask & 1:
        x = np.broadcast_to(f(x, axis=1, keepdims=True), x.shape)
    if mask & 2:
        x = np.broadcast_to(f(x, axis=0, keepdims=True), x.shape)
    return np.array(x)


def reduce_into(m: np.ndarray, mask: int, combine: str, dst_rows: int, dst_cols: int) -> np.ndarray:
    """coopmat_reduce into a dst_rows x dst_cols destination (coopmat2 flexible dimensions,
    src/device/coopmat_intrinsics.jl:685-720): Row (1) keeps m's rows and repeats each row's
    combination across the destination's columns, Column (2) the transpose of that, RowAndColumn
    (3) fills the destination with the combination of all of m.  fp32 values, combined in fp64
    (exact for the integer-valued tiles the tests use, and for max / min)."""
    R, C = m.shape
    f = {"add": np.sum, "max": np.max, "min": np.min}[combine]
    x = m.astype(np.float64)
    if mask == 1:
        assert dst_rows == R
        return np.repeat(f(x, axis=1)[:, None], dst_cols, axis=1)
    if mask == 2:
        assert dst_cols == C
        return np.repeat(f(x, axis=0)[None, :], dst_rows, axis=0)
    assert mask == 3
    return np.full((dst_rows, dst_cols), f(x))


def reduce_2x2(m: np.ndarray, combine: str) -> np.ndarray:
    """The TwoByTwo reduce (the 2 x 2 block form of SPV_NV_cooperative_matrix2; the reference
    declares the mask bit, src/vocabulary/coopmat.jl:289-297): element (i, j) of the
    (R / 2) x (C / 2) result is f(f(m[2i, 2j], m[2i, 2j+1]), f(m[2i+1, 2j], m[2i+1, 2j+1])), in fp32
    in that order."""
    x = np.asarray(m, dtype=np.float32)
    f = {"add": np.add, "max": np.maximum, "min": np.minimum}[combine]
    R, C = x.shape
    out = np.empty((R // 2, C // 2), dtype=np.float32)
    for i in range(R // 2):
        for j in range(C // 2):
            top = f(x[2 * i, 2 * j], x[2 * i, 2 * j + 1])
            bot = f(x[2 * i + 1, 2 * j], x[2 * i + 1, 2 * j + 1])
            out[i, j] = f(np.float32(top), np.float32(bot))
    return out


def load_tile(buf: np.ndarray, off: int, stride: int, rowmajor: bool, R: int, C: int) -> np.ndarray:
    """coopmat_load of an R x C tile at 0-based element offset `off`: element (r, c) at
    off + r*stride + c (RowMajor) or off + c*stride + r (ColumnMajor, the default); a
    stride of 0 makes every column (ColumnMajor) or row (RowMajor) read the same vector
    (src/compiler/spirv/coopmat.jl:664-744; src/device/coopmat_intrinsics.jl:57-75,
    402-433)."""
    r = np.arange(R)[:, None]
    c = np.arange(C)[None, :]
    idx = off + (r * stride + c if rowmajor else c * stride + r)
    return np.asarray(buf)[idx]


def store_tile(buf: np.ndarray, off: int, stride: int, rowmajor: bool, m: np.ndarray) -> np.ndarray:
    """coopmat_store of tile m into a copy of buf (same addressing as load_tile)."""
    out = np.array(buf, copy=True)
    R, C = m.shape
    r = np.arange(R)[:, None]
    c = np.arange(C)[None, :]
    out[off + (r * stride + c if rowmajor else c * stride + r)] = m
    return out


def scale_columns(m: np.ndarray, s: np.ndarray, base: int) -> np.ndarray:
    """perelement f(r, c, e, s, base) = e * float(s[base + c]) in fp32: the W8A16 per-column
    dequant through `extras` (src/device/coopmat_intrinsics.jl:569-572)."""
    f = np.asarray(s, dtype=np.float32)[base:base + m.shape[1]]
    return (np.asarray(m, dtype=np.float32) * f[None, :]).astype(np.float32)


def scale_rows(m: np.ndarray, cs: np.ndarray, base: int) -> np.ndarray:
    """perelement f(r, c, e, cs, base) = e * cs[base + r] in fp32: attention's rescale
    `element * cs[base + row]` (src/device/coopmat_intrinsics.jl:569-572)."""
    f = np.asarray(cs, dtype=np.float32)[base:base + m.shape[0]]
    return (np.asarray(m, dtype=np.float32) * f[:, None]).astype(np.float32)


# ---- GEMM epilogue ----------------------------------------------------------------------------
def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))), fp64."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def gelu_erf(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + erf(x / sqrt 2)), fp64 (math.erf per element)."""
    x = np.asarray(x, dtype=np.float64)
    erf = np.frompyfunc(math.erf, 1, 1)
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)).astype(np.float64))


ACTS = {"none": lambda x: x, "relu": lambda x: np.maximum(x, 0.0), "gelu_tanh": gelu_tanh, "gelu_erf": gelu_erf}


def gemm_epilogue(c: np.ndarray, bias=None, residual=None, act: str = "none") -> np.ndarray:
    """D = act(C + (bias[row] + residual)) in fp64, C = A*B.  The accumulator init is
    Lava's `accinit`: bias loaded at stride 0 (one value per row, every column reading
    the same vector) plus the residual, summed with coopmat_add
    (src/device/coopmat_intrinsics.jl:435-464); act is the elementwise getcomp/setcomp
    epilogue (:322-400)."""
    init = np.zeros(c.shape, dtype=np.float64)
    if bias is not None:
        init = init + np.asarray(bias, dtype=np.float64)[:, None]
    if residual is not None:
        init = init + np.asarray(residual, dtype=np.float64)
    return ACTS[act](np.asarray(c, dtype=np.float64) + init)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp64 -> fp32 -> dtype (RNE at each step, coopmat_convert of the fp32 accumulator,
    src/compiler/spirv/coopmat.jl:783-824), returned as fp64 values."""
    x32 = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x32.astype(np.float64)
    if dtype == "f16":
        return x32.astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x32)).astype(np.float64)
    raise ValueError(dtype)


# ---- tensor addressing (src/vocabulary/tensor.jl:44-108; src/device/tensor_intrinsics.jl:
# 139-155 clamp value, 258-320 load, 329-402 store), element by element.
CLAMP_UNDEFINED, CLAMP_CONSTANT, CLAMP_TO_EDGE = 0, 1, 2


def _tensor_outer(l: dict):
    """Offset of the slice's outer (rank > 2) block and whether it lies in the tensor."""
    o, inside = 0, True
    for d in range(l["rank"] - 2):
        t = l["off"][d]
        if l["clamp"] == CLAMP_TO_EDGE and l["dim"][d] > 0:
            t = min(max(t, 0), l["dim"][d] - 1)
        inside = inside and 0 <= t < l["dim"][d]
        o += t * l["stride"][d]
    return o, inside


def _tensor_elem(l: dict, outer: int, outer_in: bool, i0: int, i1: int):
    """(offset, inside) of slice element (i0, i1) of the last two dimensions, or None
    when it lies outside the slice."""
    d0, d1 = l["rank"] - 2, l["rank"] - 1
    if i0 >= l["size"][d0] or i1 >= l["size"][d1]:
        return None
    t0, t1 = l["off"][d0] + i0, l["off"][d1] + i1
    inside = outer_in and 0 <= t0 < l["dim"][d0] and 0 <= t1 < l["dim"][d1]
    if not inside and l["clamp"] == CLAMP_TO_EDGE and outer_in and l["dim"][d0] > 0 and l["dim"][d1] > 0:
        t0 = min(max(t0, 0), l["dim"][d0] - 1)
        t1 = min(max(t1, 0), l["dim"][d1] - 1)
        inside = True
    return outer + t0 * l["stride"][d0] + t1 * l["stride"][d1], inside


def tensor_load(obj: np.ndarray, src: np.ndarray, l: dict, clamp_value, transpose: bool = False) -> np.ndarray:
    """tensor_load(obj, src, layout[, view]): matrix element (r, c) is slice element
    (r, c), or (c, r) through the transposing view; outside the slice it keeps obj's
    value; inside the slice but outside the tensor it reads `clamp_value` (CONSTANT),
    the nearest element (TO_EDGE) or keeps obj's value (UNDEFINED).  `src` is the flat
    memory the layout addresses."""
    out = obj.copy()
    outer, outer_in = _tensor_outer(l)
    for r in range(obj.shape[0]):
        for c in range(obj.shape[1]):
            e = _tensor_elem(l, outer, outer_in, c if transpose else r, r if transpose else c)
            if e is None:
                continue
            if e[1]:
                out[r, c] = src[e[0]]
            elif l["clamp"] != CLAMP_UNDEFINED:
                out[r, c] = clamp_value
    return out


def tensor_store(m: np.ndarray, dst: np.ndarray, l: dict, transpose: bool = False) -> np.ndarray:
    """tensor_store(m, dst, layout[, view]): writes the elements inside both the slice and
    the tensor (a clamping store never clamps to the edge); returns the new memory."""
    out = dst.copy()
    ls = dict(l, clamp=CLAMP_CONSTANT)
    outer, outer_in = _tensor_outer(ls)
    for r in range(m.shape[0]):
        for c in range(m.shape[1]):
            e = _tensor_elem(ls, outer, outer_in, c if transpose else r, r if transpose else c)
            if e is not None and e[1]:
                out[e[0]] = m[r, c]
    return out


def rel_frobenius(x: np.ndarray, ref: np.ndarray) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / (den if den > 0 else 1.0))


def num_threads() -> int:
    return int(lib().oracle_num_threads())
