"""Ragged extents through the fast TN kernel, against the oracle.

Lava makes an extent that does not divide the tile legal with a
TENSOR_CLAMP_CONSTANT layout (src/vocabulary/tensor.jl:44-51): loads outside the
tensor read the clamp value (zero by default) and the clamping store writes only
the elements inside it (src/device/tensor_intrinsics.jl, `lava_tensor_store`).
Here A row-major and B column-major with any M and N, and K a multiple of the
16-byte chunk, take the 256 x 256 TN kernel: out-of-range lanes read zero, the
store is bounds-checked.  These tests pin the tile kernel (the dispatch rule sends
some of these shapes to the small-product kernel) and check that it ran.  Checked:
  * every row (or, for the larger shapes, edge rows plus a sample) against the
    oracle: rel. Frobenius <= 1e-3 for f16/bf16, bit-exact for int8;
  * C with padded rows (ldc > N, not a multiple of 4 -> element stores) and guard
    rows after the last: nothing outside the M x N block changes;
  * the fused epilogue on ragged shapes (bias + residual + gelu, narrowed output).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

TOL = 1e-3

# (M, N, K): ragged M, N, K; K one chunk; full M/N tiles with a ragged K; tiles of one row
SHAPES_16 = [(1000, 777, 520), (300, 4097, 64), (4095, 257, 8), (256, 256, 72), (257, 512, 1032), (513, 300, 200)]
SHAPES_I8 = [(1000, 777, 528), (300, 4097, 64), (4095, 257, 16), (256, 256, 144), (257, 512, 1040)]


def host_flat(a):
    return a.to_numpy().ravel(order=a.order)


def sample_rows(M, rng):
    edge = [0, 1, 255, 256, 257, M - 2, M - 1]
    rows = sorted({r for r in edge if 0 <= r < M} | set(rng.integers(0, M, size=min(M, 24)).tolist()))
    return np.array(rows, dtype=np.int64)


def fill(lh, a, dt, seed):
    if dt == "i8":
        lh.fill_i8(a, seed)
    else:
        lh.fill_uniform(a, seed, -1.0, 1.0)


def check(oracle, dt, got, A, B, M, N, K, lda, ldb, rows):
    if dt == "i8":
        ref = oracle.gemm_i8_rows(host_flat(A), host_flat(B), N, K, lda, ldb, 1, rows)
        np.testing.assert_array_equal(got, ref)
    else:
        ref = oracle.gemm_rows(host_flat(A), dt, host_flat(B), dt, M, N, K, lda, ldb, 1, rows)
        err = oracle.rel_frobenius(got, ref)
        assert err <= TOL, err


@pytest.mark.parametrize("crow", [True, False])
@pytest.mark.parametrize("dt,shape", [("f16", s) for s in SHAPES_16] + [("bf16", s) for s in SHAPES_16[:4]]
                         + [("i8", s) for s in SHAPES_I8])
def test_tn_ragged(gpu, oracle, tile_kernel, dt, shape, crow):
    """A row-major, B column-major; C row-major (the TN kernel as is) or column-major
    (computed as C^T = B^T A^T, so the ragged extents swap roles)."""
    lh = gpu
    M, N, K = shape
    announce(f"tn ragged {dt} M={M} N={N} K={K} C {'row' if crow else 'col'}-major")
    A = lh.HIPDeviceArray(dt, (M, K), order="C")
    B = lh.HIPDeviceArray(dt, (K, N), order="F")
    fill(lh, A, dt, 5000 + M)
    fill(lh, B, dt, 6000 + N)
    C = lh.HIPDeviceArray("i32" if dt == "i8" else "f32", (M, N), order="C" if crow else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    rows = sample_rows(M, np.random.default_rng(M * 7 + N))
    check(oracle, dt, C.to_numpy()[rows], A, B, M, N, K, K, K, rows)


@pytest.mark.parametrize("dt", ["bf16", "i8"])
def test_tn_ragged_store_stays_inside(gpu, oracle, tile_kernel, dt):
    """C row-major with ldc = N + 3 (rows not 16-byte aligned: element stores) inside a
    buffer with two guard rows: the padding columns and the guard rows keep their bytes."""
    lh = gpu
    M, N, K = 700, 601, 256 if dt == "bf16" else 512
    ldc = N + 3
    announce(f"tn ragged store bounds {dt} M={M} N={N} K={K} ldc={ldc}")
    A = lh.HIPDeviceArray(dt, (M, K), order="C")
    B = lh.HIPDeviceArray(dt, (K, N), order="F")
    fill(lh, A, dt, 7100)
    fill(lh, B, dt, 7101)
    acc = "i32" if dt == "i8" else "f32"
    Cbuf = lh.HIPDeviceArray(acc, (M + 2, ldc), order="C")
    Cbuf.fill_bytes(0x5A)
    lh.gemm_raw(dt, acc, A.ptr, B.ptr, Cbuf.ptr, M, N, K, K, K, ldc, 1 | 4)
    full = Cbuf.to_numpy().view(np.uint32)
    assert np.all(full[:, N:] == 0x5A5A5A5A), "padding columns written"
    assert np.all(full[M:, :] == 0x5A5A5A5A), "guard rows written"
    got = Cbuf.to_numpy()[:M, :N]
    rows = np.arange(M)
    check(oracle, dt, got, A, B, M, N, K, K, K, rows)


@pytest.mark.parametrize("d,crow", [("bf16", True), ("f16", False), ("f32", True)])
def test_tn_ragged_epilogue(gpu, oracle, tile_kernel, d, crow):
    """bias + residual + gelu_tanh on a ragged TN shape, narrowed to D's type."""
    lh = gpu
    M, N, K = 515, 389, 136
    announce(f"tn ragged epilogue -> {d} M={M} N={N} K={K} D {'row' if crow else 'col'}-major")
    A = lh.HIPDeviceArray("bf16", (M, K), order="C")
    B = lh.HIPDeviceArray("bf16", (K, N), order="F")
    lh.fill_uniform(A, 7200, -1.0, 1.0)
    lh.fill_uniform(B, 7201, -1.0, 1.0)
    order = "C" if crow else "F"
    D = lh.HIPDeviceArray(d, (M, N), order=order)
    D.fill_bytes(0xFF)
    bias = lh.HIPDeviceArray("f32", (M,))
    res = lh.HIPDeviceArray("f32", (M, N), order=order)
    lh.fill_uniform(bias, 7202, -1.0, 1.0)
    lh.fill_uniform(res, 7203, -2.0, 2.0)
    lh.gemm_ex(D, A, B, bias=bias, residual=res, act="gelu_tanh")
    c = oracle.gemm_rows(host_flat(A), "bf16", host_flat(B), "bf16", M, N, K, K, K, 1, np.arange(M))
    ref = oracle.round_to(oracle.gemm_epilogue(c, bias.to_numpy(), res.to_numpy(), "gelu_tanh"), d)
    h = D.to_numpy()
    got = oracle.bf16_bits_to_f32(h).astype(np.float64) if d == "bf16" else h.astype(np.float64)
    err = oracle.rel_frobenius(got, ref)
    assert err <= TOL, err


LAYOUT_SHAPES = [(512, 768, 256), (1000, 776, 520), (264, 1032, 8), (2048, 256, 1000)]


@pytest.mark.parametrize("shape", LAYOUT_SHAPES)
@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_tile_kernel_every_layout(gpu, oracle, tile_kernel, dt, layout, shape):
    """16-bit operands in all 8 layouts at sizes the 256 x 256 tile kernel takes: a
    K-contiguous operand (A row-major, B column-major) is read directly, an M/N-contiguous
    one (A column-major, B row-major) through transposing LDS reads; column-major C swaps
    the operands.  Whole tiles (512 x 768 x 256) and ragged M, N, K."""
    lh = gpu
    M, N, K = shape
    announce(f"tile kernel {dt} layout={layout} M={M} N={N} K={K}")
    A = lh.HIPDeviceArray(dt, (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray(dt, (K, N), order="C" if layout & 2 else "F")
    fill(lh, A, dt, 9000 + 10 * layout + M)
    fill(lh, B, dt, 9500 + 10 * layout + N)
    C = lh.HIPDeviceArray("f32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    rows = sample_rows(M, np.random.default_rng(layout * 131 + M))
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    ref = oracle.gemm_rows(host_flat(A), dt, host_flat(B), dt, M, N, K, lda, ldb, layout & 3, rows)
    err = oracle.rel_frobenius(C.to_numpy()[rows], ref)
    assert err <= TOL, err


@pytest.mark.parametrize("layout", [0, 2, 3, 6])
def test_tile_kernel_layouts_epilogue(gpu, oracle, tile_kernel, layout):
    """The fused epilogue on the M/N-contiguous forms (bias + residual + gelu, bf16 out)."""
    lh = gpu
    M, N, K = 520, 784, 264
    announce(f"tile kernel epilogue layout={layout}")
    A = lh.HIPDeviceArray("bf16", (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray("bf16", (K, N), order="C" if layout & 2 else "F")
    lh.fill_uniform(A, 9900 + layout, -1.0, 1.0)
    lh.fill_uniform(B, 9950 + layout, -1.0, 1.0)
    order = "C" if layout & 4 else "F"
    D = lh.HIPDeviceArray("bf16", (M, N), order=order)
    bias = lh.HIPDeviceArray("f32", (M,))
    res = lh.HIPDeviceArray("f32", (M, N), order=order)
    lh.fill_uniform(bias, 9960, -1.0, 1.0)
    lh.fill_uniform(res, 9961, -2.0, 2.0)
    lh.gemm_ex(D, A, B, bias=bias, residual=res, act="gelu_tanh")
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    c = oracle.gemm_rows(host_flat(A), "bf16", host_flat(B), "bf16", M, N, K, lda, ldb, layout & 3, np.arange(M))
    ref = oracle.round_to(oracle.gemm_epilogue(c, bias.to_numpy(), res.to_numpy(), "gelu_tanh"), "bf16")
    got = oracle.bf16_bits_to_f32(D.to_numpy()).astype(np.float64)
    err = oracle.rel_frobenius(got, ref)
    assert err <= TOL, err


@pytest.mark.parametrize("layout", range(8))
def test_tile_kernel_padded_leading_dims(gpu, oracle, tile_kernel, layout):
    """Leading dimensions larger than the extents (every operand padded by 8 elements,
    C by 4): the tile kernel's operand forms address through lda / ldb / ldc, and the
    padding of C is not written."""
    lh = gpu
    M, N, K = 520, 776, 264
    announce(f"tile kernel padded lds layout={layout}")
    arow, brow, crow = layout & 1, layout & 2, layout & 4
    lda = (K if arow else M) + 8
    ldb = (N if brow else K) + 8
    ldc = (N if crow else M) + 4
    A = lh.HIPDeviceArray("bf16", ((M if arow else K) * lda,))
    B = lh.HIPDeviceArray("bf16", ((K if brow else N) * ldb,))
    Cb = lh.HIPDeviceArray("f32", ((M if crow else N) * ldc,))
    lh.fill_uniform(A, 9700 + layout, -1.0, 1.0)
    lh.fill_uniform(B, 9800 + layout, -1.0, 1.0)
    Cb.fill_bytes(0x5A)
    lh.gemm_raw("bf16", "f32", A.ptr, B.ptr, Cb.ptr, M, N, K, lda, ldb, ldc, layout)
    rows = sample_rows(M, np.random.default_rng(layout + 77))
    ref = oracle.gemm_rows(A.to_numpy(), "bf16", B.to_numpy(), "bf16", M, N, K, lda, ldb, layout & 3, rows)
    c = Cb.to_numpy()
    cm = c.reshape(M, ldc) if crow else c.reshape(N, ldc).T
    err = oracle.rel_frobenius(cm[rows, :N] if crow else cm[:M][rows], ref)
    assert err <= TOL, err
    pad = cm[:, N:] if crow else cm[M:, :]
    assert np.all(pad.view(np.uint32) == 0x5A5A5A5A), "padding of C written"
