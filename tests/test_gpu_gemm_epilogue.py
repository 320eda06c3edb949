"""The fused GEMM epilogue family on the GPU against the oracle.

D = act(A*B + (bias + residual)) narrowed to D's type: Lava's `accinit` (bias at
stride 0, one value per row, plus the residual, src/device/coopmat_intrinsics.jl:
435-464), an elementwise getcomp/setcomp epilogue (relu, gelu in its tanh and erf
forms) and coopmat_convert to fp16 / bf16 (RNE).  The reference is the fp64 product
of the same rounded inputs, the epilogue in fp64, rounded to D's type; the bar is
the GEMM's relative Frobenius error <= 1e-3.  Covered: the fast TN kernel (A
row-major, B column-major, 256-multiples) and, through the staged kernel, every
layout with ragged extents; a column-major D exercises the transposed dispatch, in
which the bias runs along the other axis.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

TOL = 1e-3
ACTS = ["none", "relu", "gelu_tanh", "gelu_erf"]


def host_flat(a):
    return a.to_numpy().ravel(order=a.order)


def as_f64(a, oracle):
    h = a.to_numpy()
    if a.dtype == "bf16":
        return oracle.bf16_bits_to_f32(h).astype(np.float64)
    return h.astype(np.float64)


def run_case(lh, oracle, ab, d, M, N, K, layout, act, with_bias, with_res, seed):
    A = lh.HIPDeviceArray(ab, (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray(ab, (K, N), order="C" if layout & 2 else "F")
    dorder = "C" if layout & 4 else "F"
    D = lh.HIPDeviceArray(d, (M, N), order=dorder)
    lh.fill_uniform(A, seed, -1.0, 1.0)
    lh.fill_uniform(B, seed + 1, -1.0, 1.0)
    D.fill_bytes(0xFF)
    bias = res = None
    if with_bias:
        bias = lh.HIPDeviceArray("f32", (M,))
        lh.fill_uniform(bias, seed + 2, -1.0, 1.0)
    if with_res:
        res = lh.HIPDeviceArray("f32", (M, N), order=dorder)
        lh.fill_uniform(res, seed + 3, -2.0, 2.0)
    lh.gemm_ex(D, A, B, bias=bias, residual=res, act=act)
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    c = oracle.gemm_rows(host_flat(A), ab, host_flat(B), ab, M, N, K, lda, ldb, layout & 3, np.arange(M))
    ref = oracle.gemm_epilogue(c, bias.to_numpy() if bias is not None else None,
                               res.to_numpy() if res is not None else None, act)
    ref = oracle.round_to(ref, d)
    got = as_f64(D, oracle)
    err = oracle.rel_frobenius(got, ref)
    assert err <= TOL, (err, ab, d, act, with_bias, with_res, layout)
    return err


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("d", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("ab", ["f16", "bf16"])
def test_gemm_ex_tn_bias_residual(gpu, oracle, tile_kernel, ab, d, act):
    """The fast kernel with both accumulator-init terms, every output type and activation."""
    announce(f"gemm_ex TN {ab}->{d} act={act} bias+residual")
    run_case(gpu, oracle, ab, d, 256, 512, 256, 1 | 4, act, True, True, 3000)


@pytest.mark.parametrize("with_bias,with_res", [(False, False), (True, False), (False, True)])
def test_gemm_ex_tn_init_terms(gpu, oracle, tile_kernel, with_bias, with_res):
    """Each accumulator-init term alone (and neither: a plain GEMM narrowed to bf16)."""
    announce(f"gemm_ex TN bias={with_bias} residual={with_res}")
    run_case(gpu, oracle, "bf16", "bf16", 512, 256, 384, 1 | 4, "gelu_tanh", with_bias, with_res, 3100)


@pytest.mark.parametrize("d", ["f32", "bf16"])
def test_gemm_ex_column_major_d(gpu, oracle, tile_kernel, d):
    """D column-major: computed as D^T by the TN kernel, the per-row bias then runs
    along the kernel's columns and the residual is read transposed."""
    announce(f"gemm_ex column-major D -> {d}")
    run_case(gpu, oracle, "bf16", d, 256, 256, 128, 2, "relu", True, True, 3200)


@pytest.mark.parametrize("layout", range(8))
def test_gemm_ex_staged_ragged(gpu, oracle, staged_kernel, layout):
    """Ragged extents, every layout: the staged kernel with the epilogue and bounds."""
    announce(f"gemm_ex staged ragged layout={layout}")
    run_case(gpu, oracle, "f16", "f16", 100, 70, 50, layout, "gelu_erf", True, True, 3300 + 10 * layout)


def test_gemm_ex_matches_plain_gemm(gpu, oracle):
    """No init, no activation, fp32 D: the same kernel path as the plain entry point."""
    lh = gpu
    announce("gemm_ex == gemm")
    A = lh.HIPDeviceArray("bf16", (256, 256), order="C")
    B = lh.HIPDeviceArray("bf16", (256, 256), order="F")
    lh.fill_uniform(A, 3400, -1.0, 1.0)
    lh.fill_uniform(B, 3401, -1.0, 1.0)
    C1 = lh.HIPDeviceArray("f32", (256, 256), order="C")
    C2 = lh.HIPDeviceArray("f32", (256, 256), order="C")
    lh.gemm(C1, A, B)
    lh.gemm_ex(C2, A, B)
    np.testing.assert_array_equal(C1.to_numpy(), C2.to_numpy())


def test_gemm_ex_argument_errors(gpu):
    lh = gpu
    A = lh.HIPDeviceArray("f16", (16, 16), order="C")
    B = lh.HIPDeviceArray("f16", (16, 16), order="F")
    D = lh.HIPDeviceArray("f32", (16, 16), order="C")
    with pytest.raises(lh.InvalidArgument):
        lh.gemm_ex_raw("f16", "f32", A.ptr, B.ptr, D.ptr, 16, 16, 16, 16, 16, 16, 5, residual=D.ptr, ldr=8)
    with pytest.raises(ValueError):
        lh.gemm_ex(D, A, B, act="swish")
