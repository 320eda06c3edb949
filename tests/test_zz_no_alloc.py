"""The W8A16 entry point that allocates nothing, through the C ABI: the same results as
lava_hip_gemm_w8a16 (bit for bit: the same kernels and summation order) on two calls in a
row, the second smaller, and on shapes that need no split-K scratch at all (column-major
weights run one kernel over whole columns)."""
from __future__ import annotations

import numpy as np
import pytest

import lava_hip as lh_mod
from conftest import announce

pytestmark = pytest.mark.gpu


def _inputs(lh, M, N, K, cfg):
    X = lh.HIPDeviceArray("f16", (M, K), order="C")
    W = lh.HIPDeviceArray("i8", (K, N), order="C")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(cfg, 0))
    lh.fill_i8(W, lh_mod.seed(cfg, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(cfg, 2), 0.001, 0.02)
    return X, W, s


def _both(lh, M, N, K, cfg):
    X, W, s = _inputs(lh, M, N, K, cfg)
    Y_ref = lh.HIPDeviceArray("f32", (M, N), order="C")
    Y_na = lh.HIPDeviceArray("f32", (M, N), order="C")
    Y_na.fill_bytes(0xFF)
    lh.w8a16(Y_ref, X, W, s)
    lh._lib.call("lava_hip_gemm_w8a16_noalloc", X.ptr, W.ptr, s.ptr, Y_na.ptr, M, N, K, K, N, N, 7, None)
    lh.synchronize()
    return X, W, s, Y_ref.to_numpy(), Y_na.to_numpy()


def test_noalloc_matches_allocating_entry_twice(gpu, oracle):
    lh = gpu
    # split-K shapes (4 and 2 splits): the arrival counters and partial blocks live in the
    # static scratch; the second call is smaller and reuses the array the first one left behind
    for i, (M, N, K) in enumerate([(16, 4096, 4096), (8, 2048, 2048)]):
        announce(f"w8a16_noalloc call {i + 1}: M={M} N={N} K={K}")
        X, W, s, ref_entry, got = _both(lh, M, N, K, 40 + i)
        np.testing.assert_array_equal(got, ref_entry)
        ref = oracle.w8a16_rows(X.to_numpy(), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
        assert oracle.rel_frobenius(got, ref) <= 1e-3


def test_noalloc_without_split_and_argument_errors(gpu, oracle):
    lh = gpu
    announce("w8a16_noalloc: the headline shape (2 splits), ragged generic shape, bad arguments")
    for (M, N, K), cfg in (((16, 14336, 4096), 42), ((3, 7, 5), 43)):
        X, W, s, ref_entry, got = _both(lh, M, N, K, cfg)
        np.testing.assert_array_equal(got, ref_entry)
    with pytest.raises(lh.InvalidArgument):
        lh._lib.call("lava_hip_gemm_w8a16_noalloc", 16, 16, 16, 16, 16, 128, 256, 256, 100, 128, 7, None)


@pytest.mark.parametrize("M,xo,yo", [(16, "C", "C"), (16, "F", "F"), (5, "F", "C"),
                                     # several 16-row blocks per workgroup; M = 100 copies X row-major
                                     (32, "F", "F"), (64, "C", "C"), (100, "F", "C")])
def test_noalloc_column_major_weights(gpu, oracle, M, xo, yo):
    """W column-major (K contiguous per column): the whole-column kernel (no scratch, or the
    scratch holding a row-major copy of a column-major X whose M is not a multiple of 8); the
    no-allocation entry gives the same bits as the allocating one."""
    lh = gpu
    N, K = 4096, 4096
    announce(f"w8a16_noalloc: W column-major, M={M}, X {xo}, Y {yo}")
    X = lh.HIPDeviceArray("f16", (M, K), order=xo)
    W = lh.HIPDeviceArray("i8", (K, N), order="F")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(44, 0))
    lh.fill_i8(W, lh_mod.seed(44, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(44, 2), 0.001, 0.02)
    Y_ref = lh.HIPDeviceArray("f32", (M, N), order=yo)
    Y_na = lh.HIPDeviceArray("f32", (M, N), order=yo)
    Y_na.fill_bytes(0xFF)
    lh.w8a16(Y_ref, X, W, s)
    lh.w8a16_noalloc(Y_na, X, W, s)
    lh.synchronize()
    np.testing.assert_array_equal(Y_na.to_numpy(), Y_ref.to_numpy())
    ref = oracle.w8a16_rows(np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy()), s.to_numpy(),
                            N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(Y_na.to_numpy(), ref) <= 1e-3


@pytest.mark.parametrize("case", ["split", "x_copy"])
def test_noalloc_under_graph_capture(gpu, oracle, case):
    """The entry captured into a HIP graph on a fresh stream in global capture mode, where any
    hipMalloc in the process fails: a split-K shape (W row-major: counters and partial blocks in
    the fixed array) and a column-major X with M not a multiple of 8 (its row-major copy in the
    fixed array).  The graph, replayed three times with eager calls and synchronisations between
    the replays, gives the allocating entry's bits every time."""
    lh = gpu
    if case == "split":
        M, N, K, xo, wo = 16, 4096, 4096, "C", "C"
    else:
        M, N, K, xo, wo = 5, 4096, 2048, "F", "F"
    announce(f"w8a16_noalloc under graph capture: {case} M={M} N={N} K={K}")
    X = lh.HIPDeviceArray("f16", (M, K), order=xo)
    W = lh.HIPDeviceArray("i8", (K, N), order=wo)
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(45, 0))
    lh.fill_i8(W, lh_mod.seed(45, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(45, 2), 0.001, 0.02)
    Y_ref = lh.HIPDeviceArray("f32", (M, N), order="C")
    lh.w8a16(Y_ref, X, W, s)
    lh.synchronize()
    ref = Y_ref.to_numpy()
    st = lh.Stream()
    Y = lh.HIPDeviceArray("f32", (M, N), order="C")
    g = lh.Graph(st)
    with g.capture():
        lh.w8a16_noalloc(Y, X, W, s, stream=st.handle)
    Y_eager = lh.HIPDeviceArray("f32", (M, N), order="C")
    for rep in range(3):
        Y.fill_bytes(0xFF)
        lh.synchronize()
        g.launch()
        st.synchronize()
        np.testing.assert_array_equal(Y.to_numpy(), ref, err_msg=f"replay {rep}")
        lh.w8a16_noalloc(Y_eager, X, W, s)   # eager work on the same fixed array between replays
        lh.synchronize()
        np.testing.assert_array_equal(Y_eager.to_numpy(), ref)
    g.close()
    st.close()
    want = oracle.w8a16_rows(np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy()), s.to_numpy(),
                             N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(ref, want) <= 1e-3
