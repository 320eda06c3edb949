"""The library-owned workspace (W8A16 split-K partials, the row-major copy of a column-major X,
small-product GEMM split-K partials) under HIP graph capture and across its release paths.

A stream that captures a graph must not allocate (global capture mode makes any hipMalloc in
the process fail): its calls plan within the workspace the stream already has -- fewer or no K
splits -- and the buffer a graph captured stays alive after its stream is destroyed.
lava_hip_release_workspaces frees what the NULL stream (and streams made elsewhere) hold."""
from __future__ import annotations

import numpy as np
import pytest

import lava_hip as lh_mod
from conftest import announce

pytestmark = pytest.mark.gpu


def _w8_inputs(lh, M, N, K, cfg):
    X = lh.HIPDeviceArray("f16", (M, K), order="C")
    W = lh.HIPDeviceArray("i8", (K, N), order="C")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(cfg, 0))
    lh.fill_i8(W, lh_mod.seed(cfg, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(cfg, 2), 0.001, 0.02)
    return X, W, s


def test_w8a16_capture_without_workspace_then_with(gpu, oracle):
    """W row-major at 16 x 4096 . 4096 x 4096 (split-K when a workspace is available).  On a
    fresh stream the captured call plans with no workspace (one split); after an eager call has
    grown the stream's workspace, a second capture takes the split plan and matches the eager
    result bit for bit.  The graph still replays correctly after its stream is destroyed (the
    buffer it captured is kept), on another stream."""
    lh = gpu
    M, N, K = 16, 4096, 4096
    announce("w8a16 capture: no workspace, then the stream's workspace")
    X, W, s = _w8_inputs(lh, M, N, K, 46)
    want = oracle.w8a16_rows(X.to_numpy(), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
    st = lh.Stream()
    Y1 = lh.HIPDeviceArray("f32", (M, N), order="C")
    g1 = lh.Graph(st)
    lh.kernel_log_clear()
    with g1.capture():
        lh.w8a16(Y1, X, W, s, stream=st.handle)
    for _ in range(2):
        Y1.fill_bytes(0xFF)
        lh.synchronize()
        g1.launch()
        st.synchronize()
        assert oracle.rel_frobenius(Y1.to_numpy(), want) <= 1e-3
    # eager call: the stream's workspace grows to the split plan
    Ye = lh.HIPDeviceArray("f32", (M, N), order="C")
    lh.w8a16(Ye, X, W, s, stream=st.handle)
    st.synchronize()
    eager = Ye.to_numpy()
    assert oracle.rel_frobenius(eager, want) <= 1e-3
    Y2 = lh.HIPDeviceArray("f32", (M, N), order="C")
    g2 = lh.Graph(st)
    with g2.capture():
        lh.w8a16(Y2, X, W, s, stream=st.handle)
    other = lh.Stream()
    st.close()   # the graph's buffer must outlive the stream
    for rep in range(3):
        Y2.fill_bytes(0xFF)
        lh.synchronize()
        g2.launch(other)
        other.synchronize()
        np.testing.assert_array_equal(Y2.to_numpy(), eager, err_msg=f"replay {rep}")
        lh.w8a16(Ye, X, W, s)   # eager work between replays
        lh.synchronize()
    g1.close()
    g2.close()
    other.close()


@pytest.mark.parametrize("dt", ["bf16", "i8"])
def test_splitk_gemm_under_capture_runs_unsplit(gpu, oracle, dt):
    """512 x 512 x 4096 splits K eagerly; captured on a fresh stream it runs unsplit (no
    workspace to plan in, no allocation), replays give the same bits each time, and match the
    oracle (int8 bit-exact, and then equal to the eager split result too)."""
    lh = gpu
    M = N = 512
    K = 4096
    announce(f"split-K GEMM under capture {dt}")
    A = lh.HIPDeviceArray(dt, (M, K), order="C")
    B = lh.HIPDeviceArray(dt, (K, N), order="F")
    if dt == "i8":
        lh.fill_i8(A, lh_mod.seed(47, 0))
        lh.fill_i8(B, lh_mod.seed(47, 1))
    else:
        lh.fill_uniform(A, lh_mod.seed(47, 0), -1.0, 1.0)
        lh.fill_uniform(B, lh_mod.seed(47, 1), -1.0, 1.0)
    acc = "i32" if dt == "i8" else "f32"
    Ce = lh.HIPDeviceArray(acc, (M, N), order="C")
    lh.kernel_log_clear()
    lh.gemm(Ce, A, B)
    lh.synchronize()
    assert "splitk_sum_kernel" in lh.kernel_log(), lh.kernel_log()
    st = lh.Stream()
    C = lh.HIPDeviceArray(acc, (M, N), order="C")
    g = lh.Graph(st)
    lh.kernel_log_clear()
    with g.capture():
        lh.gemm(C, A, B, stream=st.handle)
    assert lh.kernel_log() == ["gemm_small_kernel"], lh.kernel_log()
    first = None
    for rep in range(3):
        C.fill_bytes(0xFF)
        lh.synchronize()
        g.launch()
        st.synchronize()
        got = C.to_numpy()
        if first is None:
            first = got.copy()
        np.testing.assert_array_equal(got, first, err_msg=f"replay {rep}")
        lh.gemm(Ce, A, B)
        lh.synchronize()
    rows = np.arange(0, M, 5)
    if dt == "i8":
        ref = oracle.gemm_i8_rows(A.to_numpy().ravel(), B.to_numpy().ravel(order="F"), N, K, K, K, 1, rows)
        np.testing.assert_array_equal(first[rows], ref)
        np.testing.assert_array_equal(first, Ce.to_numpy())
    else:
        ref = oracle.gemm_rows(A.to_numpy().ravel(), dt, B.to_numpy().ravel(order="F"), dt, M, N, K, K, K, 1, rows)
        assert oracle.rel_frobenius(first[rows], ref) <= 1e-3
    g.close()
    st.close()


def test_release_workspaces(gpu, oracle):
    """The NULL stream's workspaces (split-K GEMM and W8A16) are freed by
    lava_hip_release_workspaces; the next calls allocate them again and give the same bits."""
    lh = gpu
    announce("release_workspaces")
    A = lh.HIPDeviceArray("i8", (256, 4096), order="C")
    B = lh.HIPDeviceArray("i8", (4096, 256), order="F")
    lh.fill_i8(A, lh_mod.seed(48, 0))
    lh.fill_i8(B, lh_mod.seed(48, 1))
    C1 = lh.HIPDeviceArray("i32", (256, 256), order="C")
    C2 = lh.HIPDeviceArray("i32", (256, 256), order="C")
    X, W, s = _w8_inputs(lh, 16, 2048, 4096, 49)
    Y1 = lh.HIPDeviceArray("f32", (16, 2048), order="C")
    Y2 = lh.HIPDeviceArray("f32", (16, 2048), order="C")
    lh.gemm(C1, A, B)
    lh.w8a16(Y1, X, W, s)
    lh.release_workspaces()
    lh.gemm(C2, A, B)
    lh.w8a16(Y2, X, W, s)
    lh.synchronize()
    np.testing.assert_array_equal(C1.to_numpy(), C2.to_numpy())
    np.testing.assert_array_equal(Y1.to_numpy(), Y2.to_numpy())
    lh.release_workspaces()
    lh.release_workspaces()   # nothing left: a no-op
