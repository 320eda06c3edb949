"""The 128 x 128 mid-size GEMM kernel (gemm_mid_kernel), pinned with lava_hip_set_kernel_override,
against the oracle: rel. Frobenius <= 1e-3 for f16 / bf16, bit-exact for int8.

Each operand is K-contiguous (A row-major, B column-major) or M/N-contiguous (staged as rows of K
and read back through transposing LDS reads: 16-bit words or bytes).  C is
row-major or column-major (the latter computed as C^T = B^T A^T, which swaps the operands and flips
their layouts); ragged M, N and K take the zero-clamped loads (lanes past an extent read zero) and
the bounds-checked store, as on the 256 x 256 tile kernel whose staging it shares.  Checked: whole
tiles and ragged extents, a K of one 16-byte chunk, every operand layout, C row- and column-major,
a C with padded rows and guard rows after the last (nothing outside the M x N block changes), and the
fused epilogue (bias, residual, activation, fp32 / f16 / bf16 D) against the oracle's."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import announce
from test_gpu_gemm_epilogue import run_case as run_epilogue_case

pytestmark = pytest.mark.gpu

TOL = 1e-3

# (M, N, K): whole 128 x 128 tiles; ragged M, N, K; K one chunk; one tile; a tall thin product
SHAPES_16 = [(2048, 2048, 1024), (128, 128, 64), (1000, 777, 520), (300, 4097, 64), (129, 130, 136),
             (4095, 257, 8), (640, 1920, 2056)]
SHAPES_I8 = [(2048, 2048, 2048), (128, 128, 128), (1000, 777, 528), (300, 4097, 64), (129, 130, 144),
             (4095, 257, 16), (640, 1920, 2064)]


def host_flat(a):
    return a.to_numpy().ravel(order=a.order)


def sample_rows(M, rng):
    edge = [0, 1, 63, 64, 127, 128, 129, M - 2, M - 1]
    rows = sorted({r for r in edge if 0 <= r < M} | set(rng.integers(0, M, size=min(M, 24)).tolist()))
    return np.array(rows, dtype=np.int64)


def fill(lh, a, dt, seed):
    if dt == "i8":
        lh.fill_i8(a, seed)
    else:
        lh.fill_uniform(a, seed, -1.0, 1.0)


# M/N-contiguous operands: M (N) a multiple of the 8-element chunk; K a multiple of it where the
# other operand is K-contiguous, anything where both are M/N-contiguous (SHAPES_MN_K)
SHAPES_MN = [(2048, 2048, 1024), (128, 128, 64), (1000, 776, 520), (296, 4104, 72), (136, 136, 8),
             (4096, 256, 8), (640, 1920, 2056), (1024, 1536, 104)]
SHAPES_MN_K = [(136, 136, 1), (1024, 1536, 100), (1000, 776, 33)]
# int8: M (N) a multiple of 16 for an M/N-contiguous operand, K of 16 for a K-contiguous one
SHAPES_MN_I8 = [(2048, 2048, 2048), (128, 128, 128), (1008, 784, 528), (304, 4112, 80), (144, 144, 16),
                (640, 1920, 2064), (1024, 1536, 112)]
SHAPES_MN_K_I8 = [(144, 144, 1), (1024, 1536, 100), (1008, 784, 33)]


def check(oracle, dt, got, A, B, M, N, K, lda, ldb, rows, layout=1):
    if dt == "i8":
        ref = oracle.gemm_i8_rows(host_flat(A), host_flat(B), N, K, lda, ldb, layout, rows)
        np.testing.assert_array_equal(got, ref)
    else:
        ref = oracle.gemm_rows(host_flat(A), dt, host_flat(B), dt, M, N, K, lda, ldb, layout, rows)
        err = oracle.rel_frobenius(got, ref)
        assert err <= TOL, err


@pytest.mark.parametrize("crow", [True, False])
@pytest.mark.parametrize("dt,shape", [("f16", s) for s in SHAPES_16] + [("bf16", s) for s in SHAPES_16[:4]]
                         + [("i8", s) for s in SHAPES_I8])
def test_mid_kernel(gpu, oracle, mid_kernel, dt, shape, crow):
    """A row-major, B column-major; C row-major (the kernel as is) or column-major, computed as
    C^T = B^T A^T with A and B swapped: B^T is row-major, A^T column-major, K-contiguous again."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm mid {dt} M={M} N={N} K={K} C {'row' if crow else 'col'}-major")
    A = lh.HIPDeviceArray(dt, (M, K), order="C")
    B = lh.HIPDeviceArray(dt, (K, N), order="F")
    fill(lh, A, dt, 8000 + M)
    fill(lh, B, dt, 9000 + N)
    C = lh.HIPDeviceArray("i32" if dt == "i8" else "f32", (M, N), order="C" if crow else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    rows = sample_rows(M, np.random.default_rng(M * 7 + N))
    check(oracle, dt, C.to_numpy()[rows], A, B, M, N, K, K, K, rows)


@pytest.mark.parametrize("crow", [True, False])
@pytest.mark.parametrize("dt,shape,aorder,border",
                         [(dt, s, ao, bo) for ao, bo in [("F", "F"), ("C", "C"), ("F", "C")]
                          for dt, s in [("f16", s) for s in SHAPES_MN] + [("bf16", s) for s in SHAPES_MN[:5]]]
                         + [("f16", s, "F", "C") for s in SHAPES_MN_K] + [("bf16", SHAPES_MN_K[1], "F", "C")]
                         + [("i8", s, ao, bo) for ao, bo in [("F", "F"), ("C", "C"), ("F", "C")] for s in SHAPES_MN_I8]
                         + [("i8", s, "F", "C") for s in SHAPES_MN_K_I8])
def test_mid_kernel_layouts(gpu, oracle, mid_kernel, dt, shape, aorder, border, crow):
    """A column-major and / or B row-major: the operand that is M/N-contiguous (in the kernel's
    row-major C frame: A^T's and B^T's roles swap when C is column-major) is staged as rows of K and
    read back transposed.  Short K (1, 8, 16, 33, 72, 80, 100, 104, 112) leaves part of the last k-tile
    outside the matrix; M and N of 1000, 1008, 776, 784, 296, 304, 4104, 4112, 136, 144 end inside a
    128 x 128 tile."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm mid {dt} M={M} N={N} K={K} A {aorder} B {border} C {'row' if crow else 'col'}-major")
    A = lh.HIPDeviceArray(dt, (M, K), order=aorder)
    B = lh.HIPDeviceArray(dt, (K, N), order=border)
    fill(lh, A, dt, 8500 + M + K)
    fill(lh, B, dt, 8600 + N + K)
    C = lh.HIPDeviceArray("i32" if dt == "i8" else "f32", (M, N), order="C" if crow else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    rows = sample_rows(M, np.random.default_rng(M * 5 + N + K))
    lda = K if aorder == "C" else M
    ldb = N if border == "C" else K
    layout = (1 if aorder == "C" else 0) | (2 if border == "C" else 0)
    check(oracle, dt, C.to_numpy()[rows], A, B, M, N, K, lda, ldb, rows, layout)


@pytest.mark.parametrize("act", ["none", "relu", "gelu_tanh", "gelu_erf"])
@pytest.mark.parametrize("d", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("ab", ["f16", "bf16"])
def test_mid_kernel_epilogue(gpu, oracle, mid_kernel, ab, d, act):
    """The fused epilogue (lava_hip_gemm_ex) on the mid-size kernel: D = act(A B + (bias +
    residual)) narrowed to D's type, every input and output type and activation, against the
    oracle's fp64 epilogue rounded to D's type (every row)."""
    announce(f"gemm_ex mid {ab}->{d} act={act} bias+residual")
    run_epilogue_case(gpu, oracle, ab, d, 384, 256, 320, 1 | 4, act, True, True, 3500)


@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("shape", [(1000, 776, 520), (256, 1024, 64)])
def test_mid_kernel_epilogue_layouts(gpu, oracle, mid_kernel, layout, shape):
    """Every operand and D layout with ragged extents: a column-major D runs as its row-major
    transpose, where the bias runs along the columns; M, N, K end inside a tile."""
    M, N, K = shape
    announce(f"gemm_ex mid layout={layout} M={M} N={N} K={K}")
    run_epilogue_case(gpu, oracle, "bf16", "bf16", M, N, K, layout, "gelu_erf", True, True, 3600 + layout)


@pytest.mark.parametrize("with_bias,with_res", [(False, False), (True, False), (False, True)])
def test_mid_kernel_epilogue_terms(gpu, oracle, mid_kernel, with_bias, with_res):
    """Each accumulator-init term alone, and neither; N = 777 makes the residual's rows (ldr = N)
    unaligned to 16 bytes, so the terms are read by element, and the last column group ragged."""
    announce(f"gemm_ex mid bias={with_bias} residual={with_res}")
    run_epilogue_case(gpu, oracle, "f16", "f32", 1000, 777, 256, 1 | 4, "relu", with_bias, with_res, 3700)


@pytest.mark.parametrize("dt", ["bf16", "i8"])
def test_mid_kernel_store_stays_inside(gpu, oracle, mid_kernel, dt):
    """C row-major with ldc = N + 3 (rows not 16-byte aligned: element stores) inside a buffer
    with two guard rows: the padding columns and the guard rows keep their bytes."""
    lh = gpu
    M, N, K = 700, 601, 256 if dt == "bf16" else 512
    ldc = N + 3
    announce(f"gemm mid store bounds {dt} M={M} N={N} K={K} ldc={ldc}")
    A = lh.HIPDeviceArray(dt, (M, K), order="C")
    B = lh.HIPDeviceArray(dt, (K, N), order="F")
    fill(lh, A, dt, 8100)
    fill(lh, B, dt, 8101)
    acc = "i32" if dt == "i8" else "f32"
    Cbuf = lh.HIPDeviceArray(acc, (M + 2, ldc), order="C")
    Cbuf.fill_bytes(0x5A)
    lh.gemm_raw(dt, acc, A.ptr, B.ptr, Cbuf.ptr, M, N, K, K, K, ldc, 1 | 4)
    full = Cbuf.to_numpy().view(np.uint32)
    assert np.all(full[:, N:] == 0x5A5A5A5A), "padding columns written"
    assert np.all(full[M:, :] == 0x5A5A5A5A), "guard rows written"
    check(oracle, dt, Cbuf.to_numpy()[:M, :N], A, B, M, N, K, K, K, np.arange(M))


def test_mid_kernel_repeatable_and_linear(gpu, oracle, mid_kernel):
    """bf16 2048 x 2048 x 4096: two calls give the same bits, and C(A1 + A2) = C(A1) + C(A2)
    exactly (A1, A2, B multiples of 1/64 in [-1, 1], exact in bf16, whose products and partial sums
    are exact in fp32), so every element of C is checked, not only sampled rows."""
    lh = gpu
    M, N, K = 2048, 2048, 4096
    announce(f"gemm mid repeat/linearity bf16 M={M} N={N} K={K}")
    rng = np.random.default_rng(8200)
    a1 = (rng.integers(-32, 33, size=(M, K)) / 64.0).astype(np.float32)
    a2 = (rng.integers(-32, 33, size=(M, K)) / 64.0).astype(np.float32)
    b = (rng.integers(-32, 33, size=(K, N)) / 64.0).astype(np.float32)

    def bf16(x):   # exact in bf16: the high half of the fp32 bits (the low half is zero)
        bits = x.view(np.uint32)
        assert not (bits & 0xFFFF).any()
        return (bits >> 16).astype(np.uint16)

    A1 = lh.HIPDeviceArray.from_numpy(bf16(a1), "bf16", order="C")
    A2 = lh.HIPDeviceArray.from_numpy(bf16(a2), "bf16", order="C")
    A12 = lh.HIPDeviceArray.from_numpy(bf16(a1 + a2), "bf16", order="C")
    B = lh.HIPDeviceArray.from_numpy(bf16(b), "bf16", order="F")
    out = []
    for A in (A1, A2, A12, A12):
        C = lh.HIPDeviceArray("f32", (M, N), order="C")
        lh.gemm(C, A, B)
        out.append(C.to_numpy().astype(np.float64))
    np.testing.assert_array_equal(out[2], out[3])
    # each product is a sum of K exact terms (multiples of 1/4096 below 1): exact in fp32 while
    # the partial sums stay below 2^24 / 4096 = 4096, so the identity holds exactly
    np.testing.assert_array_equal(out[0] + out[1], out[2])


@pytest.mark.parametrize("dt,shape,kernel,aorder,border",
                         [("bf16", (2048, 2048, 2048), "gemm_mid_kernel", "C", "F"),
                          ("i8", (2048, 4096, 4096), "gemm_mid_kernel", "C", "F"),
                          ("bf16", (1536, 1536, 8192), "gemm_mid_kernel", "C", "F"),
                          ("bf16", (3072, 3072, 3072), "gemm_tn_kernel", "C", "F"),
                          ("i8", (4096, 4096, 4096), "gemm_tn_kernel", "C", "F"),
                          ("bf16", (1024, 1024, 8192), "splitk_sum_kernel", "C", "F"),
                          ("bf16", (2048, 2048, 2048), "gemm_mid_kernel", "F", "F"),
                          ("f16", (2048, 4096, 4096), "gemm_mid_kernel", "C", "C"),
                          ("bf16", (1536, 1536, 8192), "gemm_mid_kernel", "F", "C"),
                          ("bf16", (3072, 3072, 3072), "gemm_tn_kernel", "F", "F"),
                          ("i8", (2048, 2048, 2048), "gemm_mid_kernel", "F", "F"),
                          ("i8", (1024, 1024, 8192), "splitk_sum_kernel", "F", "F"),
                          ("i8", (1024, 1024, 8192), "splitk_sum_kernel", "C", "F"),
                          ("i8", (3072, 3072, 3072), "gemm_tn_kernel", "C", "C"),
                          ("bf16", (3072, 6144, 1024), "gemm_mid_kernel", "C", "F"),
                          ("i8", (4608, 4608, 1024), "gemm_mid_kernel", "F", "F"),
                          ("bf16", (6144, 4096, 1024), "gemm_tn_kernel", "C", "F")])
def test_mid_kernel_automatic_choice(gpu, oracle, dt, shape, kernel, aorder, border):
    """The automatic choice, in several operand layouts: the mid-size kernel from 128 tiles of 128 x
    128 while there are fewer than 144 of 256 x 256 and again from 257 to 336 of them, the tile
    kernel otherwise, the small-product kernel's K split below; each result against the oracle on
    sampled rows."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm automatic choice {dt} M={M} N={N} K={K} A {aorder} B {border}: {kernel}")
    A = lh.HIPDeviceArray(dt, (M, K), order=aorder)
    B = lh.HIPDeviceArray(dt, (K, N), order=border)
    fill(lh, A, dt, 8300 + M)
    fill(lh, B, dt, 8400 + N)
    C = lh.HIPDeviceArray("i32" if dt == "i8" else "f32", (M, N), order="C")
    lh.kernel_log_clear()
    lh.gemm(C, A, B)
    assert kernel in lh.kernel_log(), lh.kernel_log()
    rows = np.array([0, 1, 127, 128, M // 2, M - 1])
    lda = K if aorder == "C" else M
    ldb = N if border == "C" else K
    layout = (1 if aorder == "C" else 0) | (2 if border == "C" else 0)
    check(oracle, dt, C.to_numpy()[rows], A, B, M, N, K, lda, ldb, rows, layout)


@pytest.mark.parametrize("shape,kernel", [((2048, 2048, 2048), "gemm_mid_kernel"),
                                          ((2048, 4096, 1024), "gemm_mid_kernel"),
                                          ((3072, 3072, 1024), "gemm_tn_kernel")])
def test_mid_kernel_epilogue_automatic_choice(gpu, oracle, shape, kernel):
    """lava_hip_gemm_ex (bf16 -> bf16, bias + residual + gelu_tanh) takes the same automatic
    choice as the plain product; sampled rows against the oracle's fp64 epilogue."""
    lh = gpu
    M, N, K = shape
    announce(f"gemm_ex automatic choice bf16 M={M} N={N} K={K}: {kernel}")
    A = lh.HIPDeviceArray("bf16", (M, K), order="C")
    B = lh.HIPDeviceArray("bf16", (K, N), order="F")
    D = lh.HIPDeviceArray("bf16", (M, N), order="C")
    bias = lh.HIPDeviceArray("f32", (M,))
    res = lh.HIPDeviceArray("f32", (M, N), order="C")
    lh.fill_uniform(A, 8700, -1.0, 1.0)
    lh.fill_uniform(B, 8701, -1.0, 1.0)
    lh.fill_uniform(bias, 8702, -1.0, 1.0)
    lh.fill_uniform(res, 8703, -2.0, 2.0)
    lh.kernel_log_clear()
    lh.gemm_ex(D, A, B, bias=bias, residual=res, act="gelu_tanh")
    assert kernel in lh.kernel_log(), lh.kernel_log()
    rows = np.array([0, 1, 127, 128, M // 2, M - 1])
    c = oracle.gemm_rows(host_flat(A), "bf16", host_flat(B), "bf16", M, N, K, K, K, 1, rows)
    ref = oracle.round_to(oracle.gemm_epilogue(c, bias.to_numpy()[rows], res.to_numpy()[rows], "gelu_tanh"), "bf16")
    got = oracle.bf16_bits_to_f32(D.to_numpy()[rows]).astype(np.float64)
    err = oracle.rel_frobenius(got, ref)
    assert err <= TOL, err
