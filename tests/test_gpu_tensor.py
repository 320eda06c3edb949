"""Tensor addressing on the GPU against the oracle.

Lava's TensorLayout / TensorView vocabulary (src/vocabulary/tensor.jl; lowered in
src/device/tensor_intrinsics.jl), implemented in lava_tensor.hpp:
  * one fragment loaded through a layout (every fragment shape, fp16 and fp32, the
    three clamp modes, with and without the transposing view, slices smaller than the
    matrix, padded strides, rank-3 layouts) equals the oracle's element-by-element
    restatement -- exactly (a load moves bits);
  * the clamping store writes exactly slice ∩ tensor, through the view too;
  * the V-padding identity (tensor_intrinsics.jl:139-155): a product with V loaded
    through a CONSTANT layout whose clamp value is one has the row sums of P in the
    padding columns;
  * the coopmat2 GEMM (test/glsl/coopmat2_gemm_regs.comp) on ragged shapes, with C
    stored plainly and through the transposing view: fp16 result within rel.
    Frobenius 1e-3 of the fp64 product rounded to fp16.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

SHAPES = ["A16x16", "B16x16", "acc16x16", "acc32x32", "A32x16", "B16x32"]
NP = {"f16": np.float16, "f32": np.float32}


def random_layout(lh, rng, R, C, clamp, transpose, rank, dtype, clamp_value, shrink=False):
    """A layout over a tensor of random extents (rank 2 or 3), padded strides, and a
    slice at a random (possibly out-of-range) offset covering the matrix (or less)."""
    s0, s1 = (C, R) if transpose else (R, C)
    if shrink:
        s0, s1 = int(rng.integers(1, s0 + 1)), int(rng.integers(1, s1 + 1))
    d0, d1 = int(rng.integers(1, 41)), int(rng.integers(1, 41))
    ld = d1 + int(rng.choice([0, 3]))
    o0 = int(rng.integers(-20, d0 + 6))
    o1 = int(rng.integers(-20, d1 + 6))
    if rank == 2:
        dims, strides, offs, sizes = (d0, d1), (ld, 1), (o0, o1), (s0, s1)
        nmem = d0 * ld
    else:
        nb = int(rng.integers(1, 4))
        ob = int(rng.integers(-1, nb + 1))
        dims, strides, offs, sizes = (nb, d0, d1), (d0 * ld, ld, 1), (ob, o0, o1), (1, s0, s1)
        nmem = nb * d0 * ld
    l = lh.tensor_layout(rank, clamp)
    l = lh.tensor_setdim(l, dims)
    l = lh.tensor_setstride(l, strides)
    l = lh.tensor_setclampvalue(l, lh.tensor_clampbits(clamp_value, dtype))
    l = lh.tensor_slice(l, offs, sizes)
    return l, nmem


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES)
def test_tensor_load_tile(gpu, oracle, shape, dtype):
    lh = gpu
    _, R, C = lh.tensor.TILES[shape]
    rng = np.random.default_rng(2 * SHAPES.index(shape) + (dtype == "f32"))
    cases = 0
    for clamp in (lh.TENSOR_CLAMP_UNDEFINED, lh.TENSOR_CLAMP_CONSTANT, lh.TENSOR_CLAMP_TO_EDGE):
        for transpose in (False, True):
            for rank, shrink in ((2, False), (2, True), (3, False), (2, False)):
                cv = 2.5   # UNDEFINED keeps the object instead, whatever the clamp value
                l, nmem = random_layout(lh, rng, R, C, clamp, transpose, rank, dtype, cv, shrink)
                announce(f"tensor_load {shape} {dtype} clamp={clamp} T={transpose} {l}")
                mem = (rng.standard_normal(nmem) * 4).astype(NP[dtype])
                obj = (rng.standard_normal((R, C)) - 10).astype(NP[dtype])
                src = lh.HIPDeviceArray.from_numpy(mem, dtype=dtype)
                o = lh.HIPDeviceArray.from_numpy(obj, dtype=dtype, order="C")
                out = lh.HIPDeviceArray(dtype, (R, C), order="C")
                view = lh.tensor_view(rank, tuple(range(rank - 2)) + (rank - 1, rank - 2)) if transpose else None
                lh.tensor_load_tile(out, src, l, o, shape, view=view)
                want = oracle.tensor_load(obj, mem, l.as_dict(), NP[dtype](cv), transpose=transpose)
                np.testing.assert_array_equal(out.to_numpy(), want, err_msg=str(l))
                cases += 1
    assert cases == 24


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES)
def test_tensor_store_tile(gpu, oracle, shape, dtype):
    lh = gpu
    _, R, C = lh.tensor.TILES[shape]
    rng = np.random.default_rng(100 + 2 * SHAPES.index(shape) + (dtype == "f32"))
    for transpose in (False, True):
        for rank, shrink in ((2, False), (2, True), (3, False)):
            l, nmem = random_layout(lh, rng, R, C, lh.TENSOR_CLAMP_CONSTANT, transpose, rank, dtype, 0.0, shrink)
            announce(f"tensor_store {shape} {dtype} T={transpose} {l}")
            mem = np.full(nmem, -7.0, dtype=NP[dtype])
            m = rng.standard_normal((R, C)).astype(NP[dtype])
            dst = lh.HIPDeviceArray.from_numpy(mem, dtype=dtype)
            inp = lh.HIPDeviceArray.from_numpy(m, dtype=dtype, order="C")
            view = lh.tensor_view(rank, tuple(range(rank - 2)) + (rank - 1, rank - 2)) if transpose else None
            lh.tensor_store_tile(dst, inp, l, shape, view=view)
            want = oracle.tensor_store(m, mem, l.as_dict(), transpose=transpose)
            np.testing.assert_array_equal(dst.to_numpy(), want, err_msg=str(l))


@pytest.mark.parametrize("E", [10, 1, 15])
@pytest.mark.parametrize("via_view", [False, True])
def test_tensor_clamp_value_one_row_sums(gpu, oracle, E, via_view):
    """D = P V with V (16 keys x E) padded to 16 columns by a clamp value of one: D's first
    E columns are P V, the rest are the row sums of P.  With the view, V is stored as its
    transpose (E x 16) and read through PERM = (1, 0)."""
    lh = gpu
    announce(f"tensor clamp-one row sums E={E} view={via_view}")
    rng = np.random.default_rng(E)
    P = rng.random((16, 16)).astype(np.float16)
    V = (rng.random((16, E)) * 2 - 1).astype(np.float16)
    pa = lh.HIPDeviceArray.from_numpy(P, dtype="f16", order="C")
    la = lh.tensor_setdim(lh.tensor_layout(2, lh.TENSOR_CLAMP_CONSTANT), (16, 16))
    if via_view:
        vb = lh.HIPDeviceArray.from_numpy(np.ascontiguousarray(V.T).ravel(), dtype="f16")
        lb = lh.tensor_setdim(lh.tensor_layout(2, lh.TENSOR_CLAMP_CONSTANT), (E, 16))
        view = lh.tensor_view(2, (1, 0))
    else:
        vb = lh.HIPDeviceArray.from_numpy(V.ravel(), dtype="f16")
        lb = lh.tensor_setdim(lh.tensor_layout(2, lh.TENSOR_CLAMP_CONSTANT), (16, E))
        view = None
    lb = lh.tensor_setclampvalue(lb, lh.tensor_clampbits(1.0, "f16"))
    lb = lh.tensor_slice(lb, (0, 0), (16, 16))
    D = lh.HIPDeviceArray("f32", (16, 16), order="C")
    lh.tensor_muladd_16x16x16(D, pa, la, vb, lb, view_b=view)
    got = D.to_numpy().astype(np.float64)
    P64, V64 = P.astype(np.float64), V.astype(np.float64)
    np.testing.assert_allclose(got[:, :E], P64 @ V64, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got[:, E:], np.repeat(P64.sum(axis=1, keepdims=True), 16 - E, axis=1), rtol=1e-6)


@pytest.mark.parametrize("vocabulary", [False, True])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("shape", [(128, 128, 64), (200, 300, 100), (1, 1, 1), (513, 257, 1000), (1024, 768, 512),
                                   (64, 1000, 7), (1032, 520, 264)])
def test_gemm_cm2(gpu, oracle, shape, transpose, vocabulary):
    """Both forms: the tile kernel (default) and the tensor-vocabulary kernel."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm_cm2 M={M} N={N} K={K} transpose_c={transpose} vocabulary={vocabulary}")
    A = lh.HIPDeviceArray("f16", (M, K), order="C")
    B = lh.HIPDeviceArray("f16", (K, N), order="C")
    lh.fill_uniform(A, 8000 + M, -1.0, 1.0)
    lh.fill_uniform(B, 8100 + N, -1.0, 1.0)
    Cm = lh.HIPDeviceArray("f16", (N, M) if transpose else (M, N), order="C")
    Cm.fill_bytes(0xFF)
    lh.gemm_cm2(Cm, A, B, transpose=transpose, vocabulary=vocabulary)
    got = Cm.to_numpy().astype(np.float64)
    if transpose:
        got = got.T
    ref = oracle.gemm_rows(A.to_numpy().ravel(), "f16", B.to_numpy().ravel(), "f16", M, N, K, K, N, 3, np.arange(M))
    ref = oracle.round_to(ref, "f16")
    err = oracle.rel_frobenius(got, ref)
    assert err <= 1e-3, err


def test_gemm_cm2_k_zero_and_errors(gpu):
    lh = gpu
    announce("gemm_cm2 K=0 and argument errors")
    A = lh.HIPDeviceArray("f16", (130, 0), order="C")
    B = lh.HIPDeviceArray("f16", (0, 70), order="C")
    Cm = lh.HIPDeviceArray("f16", (130, 70), order="C")
    Cm.fill_bytes(0xFF)
    lh.gemm_cm2(Cm, A, B)
    assert np.all(Cm.to_numpy() == 0)
    Cm.fill_bytes(0xFF)
    lh.gemm_cm2(Cm, A, B, vocabulary=True)
    assert np.all(Cm.to_numpy() == 0)
    with pytest.raises(lh.InvalidArgument):
        lh._lib.call("lava_hip_gemm_cm2_f16", Cm.ptr, Cm.ptr, Cm.ptr, 130, 70, 16, 16, 70, 70, 4, None)
    with pytest.raises(lh.InvalidArgument):
        lh._lib.call("lava_hip_gemm_cm2_f16", Cm.ptr, Cm.ptr, Cm.ptr, 130, 70, 16, 8, 70, 70, 0, None)
    l = lh.tensor_setdim(lh.tensor_layout(2, 1), (4, 4))
    bad = l.to_c()
    bad.rank = 5
    import ctypes
    with pytest.raises(lh.InvalidArgument):
        lh._lib.call("lava_hip_tensor_load_tile", 0, 0, Cm.ptr, ctypes.byref(bad), 0, Cm.ptr, Cm.ptr, None)
