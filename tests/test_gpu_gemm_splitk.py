"""Split K on the small-product kernel, against the oracle.

Lava's GEMM is one `muladd` chain over K per output tile (src/vocabulary/coopmat.jl:196-203,
test/glsl/coopmat2_gemm_regs.comp:46-84); the product is a sum over K, so it may be formed as
partial sums over K ranges added afterwards.  Products of at most 256 64 x 64 tiles with at
least 8 K chunks of 512 bytes (16 above 128 tiles) run that way here: each K range's partial product goes to the
stream's workspace and a second kernel adds them in split order.  Checked:
  * every layout (A, B, C row- or column-major), f16 / bf16 against the oracle (rel.
    Frobenius <= 1e-3), int8 bit-exact (partials add modulo 2^32 like the accumulator);
  * a K that is not a multiple of the chunk (the last range is short) and ragged M, N;
  * repeat calls bit-identical (fixed summation order), C padding untouched, a non-default
    stream;
  * the workspace's front region (the W8A16 arrival counters) survives a split-K call: a
    W8A16 call after it gives the same bits as before it.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

TOL = 1e-3

# (M, N, K): 64 tiles x 16 chunks (8 splits); ragged M/N with a short last K range (6 splits),
# also with M and N not multiples of 4 (the sum's one-column form); one tile row of a wide
# product (4 splits); 256 tiles x 32 chunks (2 splits)
SHAPES_16 = [(512, 512, 4096), (136, 200, 3000), (130, 202, 3000), (64, 4096, 2048), (1024, 1024, 8192)]
SHAPES_I8 = [(512, 512, 8192), (136, 208, 6000), (64, 4096, 4096)]


def host_flat(a):
    return a.to_numpy().ravel(order=a.order)


def rows_for(M, seed):
    rng = np.random.default_rng(seed)
    if M <= 256:
        return np.arange(M, dtype=np.int64)
    edge = [0, 1, 63, 64, M - 1]
    return np.array(sorted(set(edge) | set(rng.integers(0, M, size=40).tolist())), dtype=np.int64)


def run(lh, dt, layout, M, N, K, seed, stream=None):
    A = lh.HIPDeviceArray(dt, (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray(dt, (K, N), order="C" if layout & 2 else "F")
    if dt == "i8":
        lh.fill_i8(A, seed)
        lh.fill_i8(B, seed + 1)
    else:
        lh.fill_uniform(A, seed, -1.0, 1.0)
        lh.fill_uniform(B, seed + 1, -1.0, 1.0)
    C = lh.HIPDeviceArray("i32" if dt == "i8" else "f32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B, stream=stream)
    return A, B, C


def check(oracle, dt, layout, A, B, C, M, N, K, rows):
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    got = C.to_numpy()[rows]
    if dt == "i8":
        ref = oracle.gemm_i8_rows(host_flat(A), host_flat(B), N, K, lda, ldb, layout & 3, rows)
        np.testing.assert_array_equal(got, ref)
    else:
        ref = oracle.gemm_rows(host_flat(A), dt, host_flat(B), dt, M, N, K, lda, ldb, layout & 3, rows)
        err = oracle.rel_frobenius(got, ref)
        assert err <= TOL, err


@pytest.mark.parametrize("shape", SHAPES_16)
@pytest.mark.parametrize("layout", range(8))
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_splitk_16bit_every_layout(gpu, oracle, dt, layout, shape):
    lh = gpu
    M, N, K = shape
    announce(f"split-K {dt} layout={layout} M={M} N={N} K={K}")
    A, B, C = run(lh, dt, layout, M, N, K, 31000 + 17 * layout + M + N)
    check(oracle, dt, layout, A, B, C, M, N, K, rows_for(M, layout + M))


@pytest.mark.parametrize("shape", SHAPES_I8)
@pytest.mark.parametrize("layout", range(8))
def test_splitk_int8_bit_exact(gpu, oracle, layout, shape):
    lh = gpu
    M, N, K = shape
    announce(f"split-K i8 layout={layout} M={M} N={N} K={K}")
    A, B, C = run(lh, "i8", layout, M, N, K, 32000 + 17 * layout + M + N)
    check(oracle, "i8", layout, A, B, C, M, N, K, rows_for(M, layout + N))


@pytest.mark.parametrize("layout", [0, 3, 4, 7])
def test_splitk_repeat_padding_stream(gpu, oracle, layout):
    """Padded leading dimensions, C padding untouched, a stream of its own, and two calls
    that give the same bits."""
    lh = gpu
    M, N, K = 264, 328, 4096
    announce(f"split-K padded/stream layout={layout}")
    arow, brow, crow = layout & 1, layout & 2, layout & 4
    lda = (K if arow else M) + 8
    ldb = (N if brow else K) + 8
    ldc = (N if crow else M) + 4
    A = lh.HIPDeviceArray("bf16", ((M if arow else K) * lda,))
    B = lh.HIPDeviceArray("bf16", ((K if brow else N) * ldb,))
    Cb = lh.HIPDeviceArray("f32", ((M if crow else N) * ldc,))
    lh.fill_uniform(A, 33000 + layout, -1.0, 1.0)
    lh.fill_uniform(B, 33100 + layout, -1.0, 1.0)
    Cb.fill_bytes(0x5A)
    st = lh.Stream()
    try:
        lh.gemm_raw("bf16", "f32", A.ptr, B.ptr, Cb.ptr, M, N, K, lda, ldb, ldc, layout, st.handle)
        st.synchronize()
        c1 = Cb.to_numpy().copy()
        lh.gemm_raw("bf16", "f32", A.ptr, B.ptr, Cb.ptr, M, N, K, lda, ldb, ldc, layout, st.handle)
        st.synchronize()
        c2 = Cb.to_numpy()
    finally:
        st.close()
    np.testing.assert_array_equal(c1.view(np.uint32), c2.view(np.uint32))
    cm = c1.reshape(M, ldc) if crow else c1.reshape(N, ldc).T
    rows = np.arange(M, dtype=np.int64)
    ref = oracle.gemm_rows(A.to_numpy(), "bf16", B.to_numpy(), "bf16", M, N, K, lda, ldb, layout & 3, rows)
    err = oracle.rel_frobenius(cm[:, :N] if crow else cm[:M], ref)
    assert err <= TOL, err
    pad = cm[:, N:] if crow else cm[M:, :]
    assert np.all(pad.view(np.uint32) == 0x5A5A5A5A), "padding of C written"


def test_splitk_keeps_w8a16_counters(gpu, oracle):
    """The split-K partials sit behind the W8A16 arrival counters in the same per-stream
    workspace: a W8A16 split-K call after a GEMM split-K call gives the same bits as before."""
    lh = gpu
    announce("split-K then W8A16 on one stream")
    M, N, K = 16, 14336, 4096   # row-major W at this width takes the W8A16 split-K path
    X = lh.HIPDeviceArray("f16", (M, K), order="C")
    W = lh.HIPDeviceArray("i8", (K, N), order="C")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, 34001)
    lh.fill_i8(W, 34002, symmetric=True)
    lh.fill_uniform(s, 34003, 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order="C")
    lh.w8a16(Y, X, W, s)
    y1 = Y.to_numpy().copy()
    A, B, C = run(lh, "bf16", 1, 512, 512, 8192, 34010)
    lh.w8a16(Y, X, W, s)
    np.testing.assert_array_equal(Y.to_numpy(), y1)
    check(oracle, "bf16", 1, A, B, C, 512, 512, 8192, np.arange(0, 512, 7, dtype=np.int64))
    ref = oracle.w8a16_rows(np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy()), s.to_numpy(),
                            N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(y1, ref) <= 1e-3
