"""GEMM kernels on the GPU against the oracle.

  * fp16/bf16: relative Frobenius error <= 1e-3 against the fp64 product of the
    same rounded inputs (the path's stated tolerance for 16-bit inputs);
  * int8 -> int32: bit-exact;
  * every layout combination and ragged extents through the staged kernel, and the
    small-product kernel (at most 16 tiles of 256 x 256) in every layout;
  * the benchmark configurations at full size: 256^3 fp16 (A, B row-major), 4096^3 and
    8192^3 bf16 (A row-major, B column-major), 4096^3 int8.  At full size the
    oracle checks sampled rows exactly and a size-independent property checks
    every element: sum_ij C_ij = sum_k (sum_i A_ik)(sum_j B_kj).
"""
from __future__ import annotations

import numpy as np
import pytest

import lava_hip as lh_mod
from conftest import announce

pytestmark = pytest.mark.gpu

TOL = 1e-3


def make_inputs(gpu, dt, M, N, K, layout, seed_a, seed_b):
    lh = gpu
    A = lh.HIPDeviceArray(dt, (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray(dt, (K, N), order="C" if layout & 2 else "F")
    if dt == "i8":
        lh.fill_i8(A, seed_a)
        lh.fill_i8(B, seed_b)
    else:
        lh.fill_uniform(A, seed_a, -1.0, 1.0)
        lh.fill_uniform(B, seed_b, -1.0, 1.0)
    return A, B


def host_flat(a):
    """Flat storage of a device array, in its own order."""
    h = a.to_numpy()
    return h.ravel(order=a.order)


def check_rows(oracle, dt, A, B, C, rows, layout):
    M, K = A.dims
    N = B.dims[1]
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    got = C.to_numpy()[rows]
    if dt == "i8":
        ref = oracle.gemm_i8_rows(host_flat(A), host_flat(B), N, K, lda, ldb, layout & 3, rows)
        np.testing.assert_array_equal(got, ref)
        return 0.0
    ref = oracle.gemm_rows(host_flat(A), dt, host_flat(B), dt, M, N, K, lda, ldb, layout & 3, rows)
    err = oracle.rel_frobenius(got, ref)
    assert err <= TOL, err
    return err


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("dt", ["f16", "bf16", "i8"])
@pytest.mark.parametrize("shape", [(100, 70, 50), (1, 1, 1), (64, 64, 64), (33, 257, 129), (16, 8, 0)])
def test_gemm_all_layouts_ragged(gpu, oracle, layout, dt, shape):
    lh = gpu
    M, N, K = shape
    announce(f"gemm {dt} layout={layout} M={M} N={N} K={K}")
    A, B = make_inputs(gpu, dt, M, N, K, layout, 100 + layout, 200 + layout)
    acc = "i32" if dt == "i8" else "f32"
    C = lh.HIPDeviceArray(acc, (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    if K == 0:
        assert np.all(C.to_numpy() == 0)
        return
    check_rows(oracle, dt, A, B, C, np.arange(M), layout)


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("dt", ["f16", "bf16", "i8"])
@pytest.mark.parametrize("shape", [(256, 256, 256), (192, 320, 1056), (16, 1024, 2048), (520, 136, 96)])
def test_gemm_small_products(gpu, oracle, layout, dt, shape):
    """Products of at most 16 tiles of 256 x 256 run on 64 x 64 tiles, K in 512-byte chunks
    with the next chunk in flight (one chunk, several, a ragged last one, and extents that are
    not tile multiples); K-contiguous operands staged as loaded, M/N-contiguous ones through
    transposing LDS reads (ds_read_b64_tr_b16 / _tr_b8).  int8 bit-exact."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm small {dt} layout={layout} M={M} N={N} K={K}")
    A, B = make_inputs(gpu, dt, M, N, K, layout, 300 + layout, 400 + layout)
    acc = "i32" if dt == "i8" else "f32"
    C = lh.HIPDeviceArray(acc, (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    # the 64 x 64 kernel, or the staged one where an M/N-contiguous operand's extent splits a
    # 16-byte chunk (int8 A column-major with M = 520): never the 256 x 256 tile kernel
    log = lh.kernel_log()
    assert "gemm_small_kernel" in log or "gemm_staged_kernel" in log, log
    rows = np.unique(np.concatenate([np.arange(0, M, 7), [M - 1]]))
    check_rows(oracle, dt, A, B, C, rows, layout)


def test_gemm_fp16_256_config(gpu, oracle):
    """fp16 256^3, A and B row-major, fp32 C; both the dispatching entry
    point and the 16x16x16 vocabulary-tile kernel."""
    lh = gpu
    announce("gemm f16 256^3 A,B row-major")
    A, B = make_inputs(gpu, "f16", 256, 256, 256, 3, lh_mod.seed(0, 0), lh_mod.seed(0, 1))
    for kernel in (lh.gemm, lh.coopmat_gemm_tiles):
        for corder in ("C", "F"):
            C = lh.HIPDeviceArray("f32", (256, 256), order=corder)
            kernel(C, A, B)
            check_rows(oracle, "f16", A, B, C, np.arange(256), 3 | (4 if corder == "C" else 0))


@pytest.mark.parametrize("layout", range(8))
def test_coopmat_tiles_layouts(gpu, oracle, layout):
    lh = gpu
    announce(f"coopmat tiles layout={layout}")
    A, B = make_inputs(gpu, "f16", 48, 80, 64, layout, 7, 8)
    C = lh.HIPDeviceArray("f32", (48, 80), order="C" if layout & 4 else "F")
    lh.coopmat_gemm_tiles(C, A, B)
    check_rows(oracle, "f16", A, B, C, np.arange(48), layout)


def full_checksum(C, A, B, dt):
    """sum(C) versus (colsum A) . (rowsum B), every element of C involved."""
    a = A.to_numpy()
    b = B.to_numpy()
    if dt == "bf16":
        from oracle import oracle as o
        a = o.bf16_bits_to_f32(a)
        b = o.bf16_bits_to_f32(b)
    if dt == "i8":
        lhs = int(C.to_numpy().astype(np.int64).sum())
        rhs = int(a.astype(np.int64).sum(axis=0) @ b.astype(np.int64).sum(axis=1))
        return lhs, rhs
    lhs = float(C.to_numpy().astype(np.float64).sum())
    rhs = float(a.astype(np.float64).sum(axis=0) @ b.astype(np.float64).sum(axis=1))
    return lhs, rhs


@pytest.mark.parametrize("dt,n", [("bf16", 4096), ("f16", 4096), ("i8", 4096), ("bf16", 8192), ("i8", 1024)])
def test_gemm_tn_full_size(gpu, oracle, dt, n):
    """A row-major, B column-major (the TN fast path), C row-major."""
    lh = gpu
    announce(f"gemm TN {dt} {n}^3")
    cfg = 1 if dt != "i8" else 2
    A, B = make_inputs(gpu, dt, n, n, n, 1, lh_mod.seed(cfg, 0), lh_mod.seed(cfg, 1))
    acc = "i32" if dt == "i8" else "f32"
    C = lh.HIPDeviceArray(acc, (n, n), order="C")
    lh.gemm(C, A, B)
    lh.synchronize()
    rng = np.random.default_rng(n)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, n - 1], rng.integers(0, n, 27)]))
    check_rows(oracle, dt, A, B, C, rows, 1 | 4)
    lhs, rhs = full_checksum(C, A, B, dt)
    if dt == "i8":
        assert lhs == rhs
    else:
        assert abs(lhs - rhs) <= 1e-3 * (abs(rhs) + n * np.sqrt(n))


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("shape", [(2048, 1536, 1024), (1280, 1024, 640), (1296, 1040, 528)])
def test_gemm_i8_tile_kernel_layouts(gpu, oracle, tile_kernel, layout, shape):
    """int8 on the tile kernel in every operand layout: M/N-contiguous operands staged as
    [k][m] and read through ds_read_b64_tr_b8 (whole tiles; ragged M and N; ragged K).
    Bit-exact on sampled rows."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm i8 tile kernel layout={layout} M={M} N={N} K={K}")
    A, B = make_inputs(gpu, "i8", M, N, K, layout, 500 + layout, 600 + layout)
    C = lh.HIPDeviceArray("i32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    rows = np.unique(np.concatenate([np.arange(0, M, 37), [1, 15, 16, 255, 256, M - 1]]))
    check_rows(oracle, "i8", A, B, C, rows, layout)


@pytest.mark.parametrize("layout", [0, 4])
def test_gemm_i8_full_size_column_major(gpu, oracle, layout):
    """int8 4096^3 with A column-major (Julia's layout), B column-major: every element of C
    through the exact checksum, sampled rows against the oracle."""
    lh = gpu
    n = 4096
    announce(f"gemm i8 {n}^3 layout={layout}")
    A, B = make_inputs(gpu, "i8", n, n, n, layout, lh_mod.seed(2, 0), lh_mod.seed(2, 1))
    C = lh.HIPDeviceArray("i32", (n, n), order="C" if layout & 4 else "F")
    lh.gemm(C, A, B)
    lh.synchronize()
    rng = np.random.default_rng(n + layout)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, n - 1], rng.integers(0, n, 11)]))
    check_rows(oracle, "i8", A, B, C, rows, layout)
    lhs, rhs = full_checksum(C, A, B, "i8")
    assert lhs == rhs


def test_gemm_tn_column_major_c_swaps_operands(gpu, oracle):
    """Column-major C with A column-major and B row-major is the TN kernel on the
    transposed problem."""
    lh = gpu
    announce("gemm bf16 512^3 layout=2 (C col-major through the swap)")
    A, B = make_inputs(gpu, "bf16", 512, 768, 256, 2, 3, 4)
    C = lh.HIPDeviceArray("f32", (512, 768), order="F")
    lh.gemm(C, A, B)
    check_rows(oracle, "bf16", A, B, C, np.arange(0, 512, 7), 2)


def test_gemm_streams_and_repeat(gpu, oracle):
    """Two launches on a user stream give identical results (deterministic)."""
    lh = gpu
    announce("gemm bf16 1024^3 on a stream, twice")
    A, B = make_inputs(gpu, "bf16", 1024, 1024, 1024, 1, 5, 6)
    # the inputs were filled on the NULL stream; a library stream is non-blocking, so it is
    # not ordered after that work without a synchronisation
    lh.synchronize()
    s = lh.Stream()
    C1 = lh.HIPDeviceArray("f32", (1024, 1024), order="C")
    C2 = lh.HIPDeviceArray("f32", (1024, 1024), order="C")
    lh.gemm(C1, A, B, stream=s.handle)
    lh.gemm(C2, A, B, stream=s.handle)
    s.synchronize()
    np.testing.assert_array_equal(C1.to_numpy(), C2.to_numpy())
    check_rows(oracle, "bf16", A, B, C1, np.arange(0, 1024, 37), 5)
