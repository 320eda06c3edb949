"""uint8 x uint8 -> uint32 GEMM (the unsigned coopmat product of test/spirv/test_coopmat_int8.jl:71-98,
whose operands carry no signed-component bits) at matrix scale, against the oracle, bit for bit.

The tile, mid-size and small-product kernels run it as a signed int8 product of the bytes flipped
by 128 plus a row-sum and column-sum correction; the tests pin the identity where it can go wrong:
every operand layout, ragged M, N and K (the zero padding of a ragged K enters the identity), the
extremes 0 and 255, a K long enough that the 32-bit sum wraps, split K (each split's partial
carries its own correction), and the one-thread-per-element kernel for what neither takes.  Each
test pins its kernel (lava_hip_set_kernel_override) or checks through the kernel log which ran."""
from __future__ import annotations

import numpy as np
import pytest

import lava_hip as lh_mod
from conftest import announce

pytestmark = pytest.mark.gpu


def _inputs(lh, M, N, K, layout, seed):
    A = lh.HIPDeviceArray("u8", (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray("u8", (K, N), order="C" if layout & 2 else "F")
    lh.fill_i8(A, lh_mod.seed(seed, 0))   # the generator's bytes: uniform over 0..255 as uint8
    lh.fill_i8(B, lh_mod.seed(seed, 1))
    return A, B


def _check(oracle, A, B, C, M, N, K, layout, rows):
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    ref = oracle.gemm_u8_rows(A.to_numpy().ravel(order=A.order), B.to_numpy().ravel(order=B.order), N, K, lda, ldb,
                              layout & 3, rows)
    np.testing.assert_array_equal(C.to_numpy()[rows], ref)


@pytest.fixture
def pin_gemm(gpu):
    """pin_gemm(choice): run this test's GEMMs on one kernel (1 tile, 2 small unsplit, 3 staged /
    one thread per element); the automatic choice is restored afterwards."""
    def pin(choice):
        gpu.set_kernel_override(gpu.FAMILY_GEMM, choice)
    yield pin
    gpu.set_kernel_override(gpu.FAMILY_GEMM, 0)


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("shape", [(512, 768, 1024), (1008, 784, 528), (256, 256, 16)])
def test_gemm_u8_tile_kernel(gpu, oracle, tile_kernel, layout, shape):
    lh = gpu
    M, N, K = shape
    announce(f"gemm u8 tile kernel layout={layout} M={M} N={N} K={K}")
    A, B = _inputs(lh, M, N, K, layout, 60 + layout)
    C = lh.HIPDeviceArray("u32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    assert "gemm_tn_kernel" in lh.kernel_log(), lh.kernel_log()
    rows = np.unique(np.concatenate([np.arange(0, M, 11), [r for r in (1, 15, 16, 255, 256, M - 1) if r < M]]))
    _check(oracle, A, B, C, M, N, K, layout, rows)


def test_gemm_u8_full_size(gpu, oracle):
    """4096^3 (the int8 configuration's shape, unsigned): sampled rows bit for bit, and every
    element through the sum of C modulo 2^32 against the closed form (row sums of A) . (column
    sums of B)."""
    lh = gpu
    M = N = K = 4096
    announce("gemm u8 4096^3")
    A, B = _inputs(lh, M, N, K, 1, 62)
    C = lh.HIPDeviceArray("u32", (M, N), order="C")
    lh.gemm(C, A, B)
    rows = np.array([0, 1, 777, 2048, 4095])
    _check(oracle, A, B, C, M, N, K, 1, rows)
    a = A.to_numpy().astype(np.uint64)
    b = B.to_numpy().astype(np.uint64)
    want = int((a.sum(axis=0) * b.sum(axis=1)).sum()) % (1 << 32)   # sum_mn C = sum_k colsum_A(k) rowsum_B(k)
    got = int(C.to_numpy().astype(np.uint64).sum()) % (1 << 32)
    assert got == want


@pytest.mark.parametrize("kernel", ["gemm_tn_kernel", "gemm_mid_kernel", "gemm_small_kernel<u8>", "splitk_sum_kernel"])
@pytest.mark.parametrize("value", [0, 255])
def test_gemm_u8_extremes_and_wrap(gpu, oracle, pin_gemm, value, kernel):
    """Every byte 0 or 255 (the extremes of the flipped encoding: -128 and 127) with K = 66064,
    where 255^2 K = 4295811600 passes 2^32: C must hold the product modulo 2^32 -- on the tile
    kernel, on the mid-size kernel, on the small kernel unsplit, and on the small kernel with K
    split (the automatic choice at this shape)."""
    lh = gpu
    M, N, K = 256, 256, 66064
    announce(f"gemm u8 extremes value={value} K={K} kernel={kernel}")
    pin_gemm({"gemm_tn_kernel": 1, "gemm_mid_kernel": 4, "gemm_small_kernel<u8>": 2, "splitk_sum_kernel": 0}[kernel])
    A = lh.HIPDeviceArray("u8", (M, K), order="C")
    B = lh.HIPDeviceArray("u8", (K, N), order="F")
    A.fill_bytes(value)
    B.fill_bytes(value)
    C = lh.HIPDeviceArray("u32", (M, N), order="C")
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    assert kernel in lh.kernel_log(), lh.kernel_log()
    want = (value * value * K) % (1 << 32)
    assert np.all(C.to_numpy() == np.uint32(want))


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("shape", [(512, 768, 1024), (1008, 784, 528), (144, 272, 16), (128, 128, 8208)])
def test_gemm_u8_mid_kernel(gpu, oracle, pin_gemm, layout, shape):
    """The mid-size kernel's unsigned form (128 x 128 tiles) in every layout: whole tiles, ragged M,
    N and K (K = 528, 8208: a last k-tile of 16 bytes, whose zero padding enters the identity), a K
    of one 16-byte chunk, against the oracle bit for bit."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm u8 mid kernel layout={layout} M={M} N={N} K={K}")
    pin_gemm(4)
    A, B = _inputs(lh, M, N, K, layout, 90 + layout)
    C = lh.HIPDeviceArray("u32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    assert "gemm_mid_kernel" in lh.kernel_log(), lh.kernel_log()
    rows = np.unique(np.concatenate([np.arange(0, M, 9), [r for r in (1, 15, 16, 127, 128, M - 1) if r < M]]))
    _check(oracle, A, B, C, M, N, K, layout, rows)


@pytest.mark.parametrize("layout,kernel", [(5, "gemm_mid_kernel"), (0, "gemm_mid_kernel"), (2, "gemm_mid_kernel")])
def test_gemm_u8_mid_size_automatic(gpu, oracle, layout, kernel):
    """2048 x 2048 x 4096 under the automatic choice (the mid-size kernel): sampled rows bit for bit,
    and every element through the sum of C modulo 2^32 against the closed form (column sums of A) .
    (row sums of B)."""
    lh = gpu
    M, N, K = 2048, 2048, 4096
    announce(f"gemm u8 {M}x{N}x{K} layout={layout} automatic")
    A, B = _inputs(lh, M, N, K, layout, 95 + layout)
    C = lh.HIPDeviceArray("u32", (M, N), order="C" if layout & 4 else "F")
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    assert kernel in lh.kernel_log(), lh.kernel_log()
    _check(oracle, A, B, C, M, N, K, layout, np.array([0, 1, 127, 128, 1024, 2047]))
    a = A.to_numpy().astype(np.uint64)
    b = B.to_numpy().astype(np.uint64)
    want = int((a.sum(axis=0) * b.sum(axis=1)).sum()) % (1 << 32)
    got = int(C.to_numpy().astype(np.uint64).sum()) % (1 << 32)
    assert got == want


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("shape", [(208, 144, 528), (16, 16, 16), (1024, 1024, 512), (64, 2048, 8192)])
def test_gemm_u8_small_kernel(gpu, oracle, pin_gemm, layout, shape):
    """The small-product kernel's unsigned form in every layout: a ragged tile grid, the reference's
    16x16x16 tile with a[l] = l % 7, b[l] = l % 5, a product the dispatch rule gives it, and a long
    K that it splits (64 x 2048 x 8192: 16 K ranges, each partial with its own correction), against
    the oracle bit for bit."""
    lh = gpu
    M, N, K = shape
    split = shape == (64, 2048, 8192)
    announce(f"gemm u8 small kernel layout={layout} M={M} N={N} K={K}")
    pin_gemm(0 if split else 2)
    A, B = _inputs(lh, M, N, K, layout, 80 + layout)
    if shape == (16, 16, 16):
        l = np.arange(256)
        A = lh.HIPDeviceArray.from_numpy((l % 7).astype(np.uint8).reshape(16, 16, order="F" if not layout & 1 else "C"),
                                         "u8", order="C" if layout & 1 else "F")
        B = lh.HIPDeviceArray.from_numpy((l % 5).astype(np.uint8).reshape(16, 16, order="F" if not layout & 2 else "C"),
                                         "u8", order="C" if layout & 2 else "F")
    C = lh.HIPDeviceArray("u32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    log = lh.kernel_log()
    assert "gemm_small_kernel<u8>" in log, log
    if split:
        assert "splitk_sum_kernel" in log, log
    rows = np.unique(np.concatenate([np.arange(0, M, 7), [M - 1]]))
    _check(oracle, A, B, C, M, N, K, layout, rows)


@pytest.mark.parametrize("layout", [0, 3, 5, 7])
@pytest.mark.parametrize("shape", [(100, 70, 50), (16, 16, 16), (300, 257, 33), (5, 1, 7)])
def test_gemm_u8_generic_kernel(gpu, oracle, pin_gemm, layout, shape):
    """The one-thread-per-element kernel (what runs where neither MFMA kernel fits: extents that split
    a 16-byte chunk, as in most of these shapes; pinned here for all of them), including the
    reference's 16x16x16 tile with a[l] = l % 7, b[l] = l % 5."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm u8 generic layout={layout} M={M} N={N} K={K}")
    pin_gemm(3)
    A, B = _inputs(lh, M, N, K, layout, 70 + layout)
    if shape == (16, 16, 16):
        l = np.arange(256)
        A = lh.HIPDeviceArray.from_numpy((l % 7).astype(np.uint8).reshape(16, 16, order="F" if not layout & 1 else "C"),
                                         "u8", order="C" if layout & 1 else "F")
        B = lh.HIPDeviceArray.from_numpy((l % 5).astype(np.uint8).reshape(16, 16, order="F" if not layout & 2 else "C"),
                                         "u8", order="C" if layout & 2 else "F")
    C = lh.HIPDeviceArray("u32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    assert lh.kernel_log() == ["gemm_u8_generic_kernel"], lh.kernel_log()
    _check(oracle, A, B, C, M, N, K, layout, np.arange(M))
