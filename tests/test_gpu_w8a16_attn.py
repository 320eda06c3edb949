"""W8A16 decode GEMM and causal flash-attention forward on the GPU, against the
oracle (rel-Frobenius <= 1e-3 and <= 2e-3, the path's stated tolerances).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import lava_hip as lh_mod
from conftest import announce

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ W8A16
def w8_inputs(lh, M, N, K, seed_cfg=3, order="C"):
    X = lh.HIPDeviceArray("f16", (M, K), order=order)
    W = lh.HIPDeviceArray("i8", (K, N), order=order)
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(seed_cfg, 0))
    lh.fill_i8(W, lh_mod.seed(seed_cfg, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(seed_cfg, 2), 0.001, 0.02)
    return X, W, s


@pytest.mark.parametrize("M,N,K", [(16, 14336, 4096), (16, 1024, 512), (5, 256, 128), (32, 384, 1024),
                                   (16, 200, 96), (3, 7, 5),
                                   # step counts that are not powers of two: 86 and 112 steps of 32
                                   # per wavefront before the split (decode shapes of common models), 3
                                   (16, 4096, 11008), (16, 4096, 14336), (1, 1024, 384), (48, 256, 1408),
                                   # K a multiple of 32 only: unequal per-wavefront shares, some empty
                                   (16, 256, 96), (7, 384, 1120), (16, 128, 32),
                                   # wide N: one split, several row blocks with uneven shares, M = 1
                                   (16, 11008, 4096), (33, 6144, 1120), (1, 10240, 64), (16, 12288, 96)])
def test_w8a16(gpu, oracle, M, N, K):
    lh = gpu
    announce(f"w8a16 M={M} N={N} K={K}")
    X, W, s = w8_inputs(lh, M, N, K)
    Y = lh.HIPDeviceArray("f32", (M, N), order="C")
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    ref = oracle.w8a16_rows(X.to_numpy(), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
    err = oracle.rel_frobenius(Y.to_numpy(), ref)
    assert err <= 1e-3, err
    # repeat: the split-K partials are summed in a fixed order, so a second call is identical
    Y2 = lh.HIPDeviceArray("f32", (M, N), order="C")
    lh.w8a16(Y2, X, W, s)
    np.testing.assert_array_equal(Y.to_numpy(), Y2.to_numpy())


@pytest.mark.parametrize("M,N,K,xo,yo", [(16, 4096, 4096, "F", "C"), (16, 4096, 4096, "C", "F"), (16, 14336, 4096, "F", "F"),
                                         (5, 256, 1024, "F", "F"), (33, 6144, 1120, "F", "C"), (1, 1024, 384, "C", "F")])
def test_w8a16_row_major_w_orders(gpu, oracle, M, N, K, xo, yo):
    """Row-major W with X and/or Y column-major: the split-K stream kernel (column-major X
    gathered with 2-byte loads, column-major Y stored column by column); repeat calls identical."""
    lh = gpu
    announce(f"w8a16 W row-major M={M} N={N} K={K} X {xo} Y {yo}")
    X = lh.HIPDeviceArray("f16", (M, K), order=xo)
    W = lh.HIPDeviceArray("i8", (K, N), order="C")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(7, 0))
    lh.fill_i8(W, lh_mod.seed(7, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(7, 2), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order=yo)
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    y1 = Y.to_numpy()
    lh.w8a16(Y, X, W, s)
    np.testing.assert_array_equal(Y.to_numpy(), y1)
    ref = oracle.w8a16_rows(np.ascontiguousarray(X.to_numpy()), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(y1, ref) <= 1e-3


@pytest.mark.parametrize("M,N,K,xo,yo", [(16, 136, 4096, "C", "C"), (16, 8, 256, "C", "C"), (5, 1000, 1024, "F", "C"),
                                         (16, 14344, 4096, "C", "C"), (1, 50264, 64, "C", "F"), (33, 2056, 1120, "F", "F"),
                                         (16, 200, 96, "C", "C"), (7, 392, 32, "C", "C")])
def test_w8a16_row_major_w_ragged_n(gpu, oracle, M, N, K, xo, yo):
    """Row-major W with N a multiple of 8 but not of 128: the split-K kernel's last column block
    reads the last 8 columns in place of those past N and stores only the columns below N (split
    and unsplit K); repeat calls identical."""
    lh = gpu
    announce(f"w8a16 W row-major ragged N M={M} N={N} K={K} X {xo} Y {yo}")
    X = lh.HIPDeviceArray("f16", (M, K), order=xo)
    W = lh.HIPDeviceArray("i8", (K, N), order="C")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(9, 0))
    lh.fill_i8(W, lh_mod.seed(9, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(9, 2), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order=yo)
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    y1 = Y.to_numpy()
    lh.w8a16(Y, X, W, s)
    np.testing.assert_array_equal(Y.to_numpy(), y1)
    ref = oracle.w8a16_rows(np.ascontiguousarray(X.to_numpy()), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(y1, ref) <= 1e-3


@pytest.mark.parametrize("M,N,K,padw,pady", [(16, 200, 512, 56, 24), (3, 1032, 4096, 8, 8)])
def test_w8a16_row_major_w_ragged_n_padding(gpu, oracle, M, N, K, padw, pady):
    """Row-major W and Y with leading dimensions past a ragged N: the columns past N of Y keep
    their bytes (no store lands there) and the weight padding is never used."""
    lh = gpu
    announce(f"w8a16 W row-major ragged N padded M={M} N={N} K={K} ldw=N+{padw} ldy=N+{pady}")
    ldw, ldy = N + padw, N + pady
    X = lh.HIPDeviceArray("f16", (M, K), order="C")
    Wp = lh.HIPDeviceArray("i8", (K, ldw), order="C")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(10, 0))
    lh.fill_i8(Wp, lh_mod.seed(10, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(10, 2), 0.001, 0.02)
    Yp = lh.HIPDeviceArray("f32", (M, ldy), order="C")
    Yp.fill_bytes(0xFF)
    lh.w8a16_raw(X.ptr, Wp.ptr, s.ptr, Yp.ptr, M, N, K, K, ldw, ldy, layout=7)
    yp = Yp.to_numpy()
    assert (yp[:, N:].view(np.uint32) == 0xFFFFFFFF).all()
    Wh = np.ascontiguousarray(Wp.to_numpy()[:, :N])
    ref = oracle.w8a16_rows(X.to_numpy(), Wh, s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(np.ascontiguousarray(yp[:, :N]), ref) <= 1e-3


def test_w8a16_two_threads_one_stream(gpu, oracle):
    """Split-K calls from two host threads on the NULL stream: each call's kernel pair is
    enqueued whole, so neither thread's partial sums are overwritten by the other's."""
    import threading
    lh = gpu
    announce("w8a16 split-K from two threads on one stream")
    shapes = [(16, 4096, 4096), (8, 2048, 8192)]
    cases = []
    for i, (M, N, K) in enumerate(shapes):
        X, W, s = w8_inputs(lh, M, N, K, seed_cfg=20 + i)
        Y = lh.HIPDeviceArray("f32", (M, N), order="C")
        lh.w8a16(Y, X, W, s)
        lh.synchronize()
        cases.append((X, W, s, Y, Y.to_numpy()))
    errors = []

    def worker(case):
        X, W, s, Y, _ = case
        try:
            for _ in range(30):
                lh.w8a16(Y, X, W, s)
        except Exception as e:   # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(c,)) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    lh.synchronize()
    assert not errors, errors
    for (M, N, K), (X, W, s, Y, first) in zip(shapes, cases):
        np.testing.assert_array_equal(Y.to_numpy(), first)
        ref = oracle.w8a16_rows(X.to_numpy(), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
        assert oracle.rel_frobenius(first, ref) <= 1e-3


def test_w8a16_stream_destroy_releases_workspace(gpu, oracle):
    """A split-K call on a library stream, then the stream destroyed (it drains first);
    a new stream gets a new workspace and the same result."""
    lh = gpu
    announce("w8a16 split-K on a stream, stream destroyed, again on another")
    M, N, K = 16, 4096, 4096
    X, W, s = w8_inputs(lh, M, N, K, seed_cfg=22)
    lh.synchronize()
    outs = []
    for _ in range(2):
        st = lh.Stream()
        Y = lh.HIPDeviceArray("f32", (M, N), order="C")
        lh.w8a16(Y, X, W, s, stream=st.handle)
        st.close()
        outs.append(Y.to_numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    ref = oracle.w8a16_rows(X.to_numpy(), W.to_numpy(), s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(outs[0], ref) <= 1e-3


@pytest.mark.parametrize("M,N,K", [(16, 14336, 4096), (1, 4096, 4096), (5, 11008, 4096), (16, 96, 64), (40, 256, 1024),
                                   (16, 4096, 11008 // 64 * 64),
                                   # K not a multiple of the 128-k stage: a partial last stage, and
                                   # K quarters of unequal length (some empty when K < 4 stages)
                                   (16, 4096, 1040), (3, 256, 48), (17, 64, 4112), (16, 32, 400),
                                   # N not a multiple of the 32-column block: a ragged last block (an LM
                                   # head with an odd vocabulary, and small N)
                                   (16, 50257, 1024), (5, 100, 256), (16, 33, 128), (1, 1, 64),
                                   # K not a multiple of 16: the generic kernel
                                   (4, 64, 40)])
def test_w8a16_weights_column_major(gpu, oracle, M, N, K):
    """W column-major (K contiguous per output column, the layout of a linear layer's weight),
    X and Y row-major: the whole-column kernel (no split-K); rows past M read as zero and
    more than one 16-row block of X; repeat calls identical."""
    w8a16_column_major_case(gpu, oracle, M, N, K, "C", "C")


@pytest.mark.parametrize("M,N,K,xo,yo", [
    # all column-major (the Julia default), X column-major only, Y column-major only
    (16, 14336, 4096, "F", "F"), (16, 4096, 4096, "F", "C"), (16, 4096, 4096, "C", "F"),
    # two row blocks, the second of 8 rows; a partial last stage
    (24, 96, 400, "F", "C"), (8, 4096, 1040, "F", "F"), (40, 256, 1024, "F", "F"),
    # one row with unit stride (read as row-major); M not a multiple of 8 (X copied row-major into
    # the workspace first)
    (1, 4096, 4096, "F", "F"), (5, 256, 128, "F", "F"), (3, 4096, 4096, "F", "C"), (7, 14336, 4096, "F", "F"),
    (12, 1024, 1040, "F", "F"), (21, 512, 256, "F", "C"),
    # four row blocks; a long K (down projection)
    (64, 2048, 4096, "F", "C"), (16, 4096, 14336, "C", "C")])
def test_w8a16_weights_column_major_orders(gpu, oracle, M, N, K, xo, yo):
    """Column-major W with X and Y in either orientation."""
    w8a16_column_major_case(gpu, oracle, M, N, K, xo, yo)


@pytest.mark.parametrize("M,N,K,xo,yo,kernel", [
    # two 16-row blocks per workgroup (the second partial); row- and column-major X
    (17, 2048, 1024, "C", "C", "w8a16_kmajor_kernel<mb2>"), (32, 2048, 4096, "F", "F", "w8a16_kmajor_kernel<mb2>"),
    # four: a partial group of three blocks, a ragged last stage, the headline N, two and four groups
    (33, 1024, 1040, "C", "F", "w8a16_kmajor_kernel<mb4>"), (48, 4096, 4096, "F", "C", "w8a16_kmajor_kernel<mb4>"),
    (64, 14336, 4096, "C", "C", "w8a16_kmajor_kernel<mb4>"), (128, 4096, 4096, "F", "F", "w8a16_kmajor_kernel<mb4>"),
    (256, 2048, 4096, "C", "C", "w8a16_kmajor_kernel<mb4>"),
    # M not a multiple of 8 with X column-major: X copied row-major first, a last group of one row
    (65, 512, 4096, "F", "F", "w8a16_kmajor_kernel<mb4>"), (100, 2048, 2048, "F", "C", "w8a16_kmajor_kernel<mb4>")])
def test_w8a16_weights_column_major_row_blocks(gpu, oracle, M, N, K, xo, yo, kernel):
    """Batches above 16 rows: each workgroup multiplies 2 or 4 row blocks of X with every
    dequantized W fragment, so W streams once per 32 or 64 rows; against the oracle, and through
    the kernel log, the row-block form that ran."""
    gpu.kernel_log_clear()
    w8a16_column_major_case(gpu, oracle, M, N, K, xo, yo)
    assert kernel in gpu.kernel_log(), gpu.kernel_log()


def w8a16_column_major_case(lh, oracle, M, N, K, xo, yo):
    announce(f"w8a16 W column-major M={M} N={N} K={K} X {xo} Y {yo}")
    X = lh.HIPDeviceArray("f16", (M, K), order=xo)
    W = lh.HIPDeviceArray("i8", (K, N), order="F")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(5, 0))
    lh.fill_i8(W, lh_mod.seed(5, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(5, 2), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order=yo)
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    y1 = Y.to_numpy()
    lh.w8a16(Y, X, W, s)
    np.testing.assert_array_equal(Y.to_numpy(), y1)
    Xh = np.ascontiguousarray(X.to_numpy())          # row-major copies for the oracle
    Wh = np.ascontiguousarray(W.to_numpy())
    rows = np.arange(M)
    ref = oracle.w8a16_rows(Xh, Wh, s.to_numpy(), N, K, K, N, rows)
    assert oracle.rel_frobenius(y1, ref) <= 1e-3


@pytest.mark.parametrize("M,N,K,padx,padw", [(16, 4096, 4096, 8, 16), (5, 256, 1040, 24, 48)])
def test_w8a16_weights_column_major_strided(gpu, oracle, M, N, K, padx, padw):
    """Column-major W and row-major X with leading dimensions past K (padding never read)."""
    lh = gpu
    announce(f"w8a16 W column-major strided M={M} N={N} K={K} ldx=K+{padx} ldw=K+{padw}")
    ldx, ldw = K + padx, K + padw
    Xp = lh.HIPDeviceArray("f16", (M, ldx), order="C")
    Wp = lh.HIPDeviceArray("i8", (ldw, N), order="F")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(Xp, lh_mod.seed(6, 0))
    lh.fill_i8(Wp, lh_mod.seed(6, 1), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(6, 2), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order="C")
    lh.w8a16_raw(Xp.ptr, Wp.ptr, s.ptr, Y.ptr, M, N, K, ldx, ldw, N, layout=5)
    Xh = np.ascontiguousarray(Xp.to_numpy()[:, :K])
    Wh = np.ascontiguousarray(Wp.to_numpy()[:K, :])
    ref = oracle.w8a16_rows(Xh, Wh, s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(Y.to_numpy(), ref) <= 1e-3


def test_w8a16_column_major_generic(gpu, oracle):
    lh = gpu
    announce("w8a16 column-major operands, K not a multiple of 16 (generic kernel)")
    M, N, K = 8, 100, 40
    X, W, s = w8_inputs(lh, M, N, K, order="F")
    Y = lh.HIPDeviceArray("f32", (M, N), order="F")
    lh.w8a16(Y, X, W, s)
    Xh, Wh = np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy())
    ref = oracle.w8a16_rows(Xh, Wh, s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(Y.to_numpy(), ref) <= 1e-3


# ------------------------------------------------------------------ attention
@pytest.fixture
def so_kernel(gpu):
    """Checks, after the test, that its calls ran on the score/output kernel (flash_fwd5_kernel),
    through the library's kernel log."""
    gpu.kernel_log_clear()
    yield
    assert "flash_fwd5_kernel" in gpu.kernel_log(), gpu.kernel_log()


def attn_inputs(lh, E, L, H, B, cfg=4):
    Q, K, V = (lh.HIPDeviceArray("f16", (E, L, H, B)) for _ in range(3))
    for t, a in enumerate((Q, K, V)):
        lh.fill_normal(a, lh_mod.seed(cfg, t))
    return Q, K, V


def check_heads(oracle, Q, K, V, O, scale, causal, heads, rows):
    E, L, H, B = Q.dims
    st = (1, E, E * L, E * L * H)
    q, k, v = (a.to_numpy().ravel(order="F") for a in (Q, K, V))
    o = O.to_numpy()
    worst = 0.0
    for (b, h) in heads:
        ref = oracle.attn_rows(q, k, v, L, E, st, scale, causal, b, h, rows)
        got = o[:, rows, h, b].T.astype(np.float64)
        err = oracle.rel_frobenius(got, ref)
        worst = max(worst, err)
        assert err <= 2e-3, (b, h, err)
    return worst


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("E,L,H,B", [(128, 128, 1, 1), (128, 512, 3, 2), (128, 1024, 2, 1)])
def test_flash_fast_path(gpu, oracle, so_kernel, causal, E, L, H, B):
    lh = gpu
    announce(f"flash fwd D={E} S={L} H={H} B={B} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, H, B)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, causal=causal)
    heads = [(b, h) for b in range(B) for h in range(H)]
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(E), causal, heads, np.arange(L))


@pytest.mark.parametrize("H,B", [(4, 2), (8, 3), (8, 4), (5, 1)])
def test_flash_causal_block_orders(gpu, oracle, so_kernel, H, B):
    """Causal workgroup orders: B * H = 8 (one head per XCD), 24 (three per XCD, no
    4-head groups), 32 (groups of 4 heads), 5 (no split by XCD); every head's rows."""
    lh = gpu
    E, L = 128, 1024
    announce(f"flash fwd causal order D={E} S={L} H={H} B={B}")
    Q, K, V = attn_inputs(lh, E, L, H, B)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, causal=True)
    heads = [(b, h) for b in range(B) for h in range(H)]
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(E), True, heads, np.arange(0, L, 7))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("L", [128, 777, 1024])
def test_flash_pingpong_kernel_d128(gpu, oracle, causal, L):
    """D = 128 on the ping-pong kernel (pinned with lava_hip_set_kernel_override; the default
    D = 128 path is the score/output split kernel), including a ragged S."""
    lh = gpu
    announce(f"flash fwd ping-pong kernel D=128 S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, 128, L, 2, 1)
    O = lh.HIPDeviceArray("f16", (128, L, 2, 1))
    O.fill_bytes(0xFF)
    lh.set_kernel_override(lh.FAMILY_ATTN, 3)
    lh.kernel_log_clear()
    try:
        lh.flash_attn_fwd(O, Q, K, V, causal=causal)
        assert lh.kernel_log() == ["flash_fwd3_kernel"], lh.kernel_log()
    finally:
        lh.set_kernel_override(lh.FAMILY_ATTN, 0)
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(128), causal, [(0, 0), (0, 1)], np.arange(L))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("L", [1, 7, 100, 255, 257, 1000, 1537])
def test_flash_fast_ragged_s(gpu, oracle, so_kernel, causal, L):
    """D = 128 with S not a multiple of the 256-query block: the fast kernel zero-fills the
    K/V rows past S (offsets beyond the buffer resource), masks their scores, computes the
    queries past S on zeros and does not store them.  Every row of every head up to S = 257,
    edge rows plus a sample beyond."""
    lh = gpu
    E, H, B = 128, 2, 2
    announce(f"flash fast ragged D={E} S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, H, B)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, causal=causal)
    if L <= 257:
        rows = np.arange(L)
    else:
        rng = np.random.default_rng(L)
        edge = [0, 1, 63, 64, 255, 256, L - 65, L - 64, L - 2, L - 1]
        rows = np.unique(np.concatenate([[r for r in edge if 0 <= r < L], rng.integers(0, L, 24)]))
    heads = [(b, h) for b in range(B) for h in range(H)]
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(E), causal, heads, rows)
    assert not np.isnan(O.to_numpy()).any()


@pytest.mark.parametrize("kernel", ["flash_fwd3_kernel", "flash_fwd5_kernel"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("L", [64, 256, 777, 2048])
def test_flash_fast_d64(gpu, oracle, causal, L, kernel):
    """Head dimension 64 on both MFMA kernels, each pinned: the ping-pong kernel (128-byte rows,
    4 S^T k-steps, 2 O^T tiles) and the score/output kernel (rows staged 128 wide, MFMAs over
    the 64 columns that hold data: 4 S^T k-steps, 2 O^T tiles)."""
    lh = gpu
    E, H, B = 64, 2, 2
    announce(f"flash fast D=64 S={L} causal={causal} {kernel}")
    Q, K, V = attn_inputs(lh, E, L, H, B)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.set_kernel_override(lh.FAMILY_ATTN, 3 if kernel == "flash_fwd3_kernel" else 5)
    lh.kernel_log_clear()
    try:
        lh.flash_attn_fwd(O, Q, K, V, causal=causal)
        assert kernel in lh.kernel_log(), lh.kernel_log()
    finally:
        lh.set_kernel_override(lh.FAMILY_ATTN, 0)
    rng = np.random.default_rng(L + 1)
    rows = np.arange(L) if L <= 256 else np.unique(np.concatenate([[0, 1, 255, 256, L - 1], rng.integers(0, L, 32)]))
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(E), causal, [(b, h) for b in range(B) for h in range(H)], rows)
    assert not np.isnan(O.to_numpy()).any()


@pytest.mark.parametrize("E,L,causal", [(20, 200, True), (100, 130, False), (164, 100, True), (250, 64, False)])
def test_flash_generic_path(gpu, oracle, E, L, causal):
    """Head dims the MFMA kernels do not take (not a multiple of 8)."""
    lh = gpu
    announce(f"flash generic D={E} S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, 2, 1)
    O = lh.HIPDeviceArray("f16", (E, L, 2, 1))
    lh.flash_attn_fwd(O, Q, K, V, scale=0.2, causal=causal)
    check_heads(oracle, Q, K, V, O, 0.2, causal, [(0, 0), (0, 1)], np.arange(L))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("L,H,B", [(64, 2, 1), (300, 2, 1), (1000, 1, 2), (2048, 2, 1)])
def test_flash_d256(gpu, oracle, causal, L, H, B):
    """D = 256: the ping-pong kernel over 512-byte Q/K rows, launched once per 128-column half
    of V and O (scores computed in each); ragged S, several heads and batches."""
    lh = gpu
    announce(f"flash D=256 S={L} H={H} B={B} causal={causal}")
    Q, K, V = attn_inputs(lh, 256, L, H, B)
    O = lh.HIPDeviceArray("f16", (256, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, causal=causal)
    rows = np.arange(L) if L <= 300 else np.unique(np.concatenate([np.arange(0, L, 13), [L - 1]]))
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(256), causal, [(b, h) for b in range(B) for h in range(H)], rows)
    assert not np.isnan(O.to_numpy()).any()


@pytest.mark.parametrize("E,L,causal", [(136, 200, True), (160, 100, False), (192, 300, True), (200, 64, False),
                                         (248, 777, True), (192, 1000, False)])
def test_flash_padded_head_dims_above_128(gpu, oracle, E, L, causal):
    """128 < D < 256 (multiples of 8) on the ping-pong kernel zero-padded to 256: the padding
    columns of Q and K read zero; the second launch covers V and O columns 128 .. D - 1 and
    writes no others."""
    lh = gpu
    announce(f"flash padded D={E} S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, 2, 1)
    O = lh.HIPDeviceArray("f16", (E, L, 2, 1))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=0.1, causal=causal)
    rows = np.arange(L) if L <= 300 else np.unique(np.concatenate([np.arange(0, L, 7), [L - 1]]))
    check_heads(oracle, Q, K, V, O, 0.1, causal, [(0, 0), (0, 1)], rows)
    assert not np.isnan(O.to_numpy()).any()


@pytest.mark.parametrize("causal", [True, False])
def test_flash_d256_nonpositive_scale(gpu, oracle, causal):
    """D = 256 with a negative scale runs on the generic kernel (the ping-pong kernel's running
    maximum assumes a positive scale)."""
    lh = gpu
    announce(f"flash D=256 scale<0 causal={causal}")
    Q, K, V = attn_inputs(lh, 256, 100, 1, 1)
    O = lh.HIPDeviceArray("f16", (256, 100, 1, 1))
    lh.flash_attn_fwd(O, Q, K, V, scale=-0.0625, causal=causal)
    check_heads(oracle, Q, K, V, O, -0.0625, causal, [(0, 0)], np.arange(100))


@pytest.mark.parametrize("E,L,causal", [(32, 200, True), (16, 32, True), (96, 130, False), (48, 100, False),
                                         (8, 257, True), (120, 300, False), (80, 512, True), (96, 1000, True)])
def test_flash_padded_head_dims(gpu, oracle, so_kernel, E, L, causal):
    """Head dimensions below 128 (multiples of 8) on the score/output kernel, staged zero-padded
    to 128 with MFMAs over D rounded up to 64, 96 or 128: the padding columns of Q and K read
    zero and add nothing to the scores; those of O are not written."""
    lh = gpu
    announce(f"flash padded D={E} S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, 2, 1)
    O = lh.HIPDeviceArray("f16", (E, L, 2, 1))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=0.2, causal=causal)
    rows = np.arange(L) if L <= 300 else np.unique(np.concatenate([np.arange(0, L, 7), [L - 1]]))
    check_heads(oracle, Q, K, V, O, 0.2, causal, [(0, 0), (0, 1)], rows)
    assert not np.isnan(O.to_numpy()).any()


def test_flash_golden(gpu, so_kernel):
    from pathlib import Path
    lh = gpu
    announce("flash golden S=32 D=16")
    g = dict(np.load(Path(__file__).resolve().parent / "golden" / "known_answers.npz"))
    Q, K, V = (lh.HIPDeviceArray.from_numpy(np.asfortranarray(g[k]), "f16") for k in ("attn_q", "attn_k", "attn_v"))
    O = lh.HIPDeviceArray("f16", Q.dims)
    lh.flash_attn_fwd(O, Q, K, V, causal=True)
    from oracle import oracle as o
    assert o.rel_frobenius(O.to_numpy(), g["attn_o"]) <= 2e-3


def test_flash_full_config(gpu, oracle, so_kernel):
    """B=4, H=32, S=4096, D=128, causal, scale 1/sqrt(128).  Sampled
    heads and rows against the oracle, plus properties of every row: causal row 0
    equals v_0 exactly (up to fp16 rounding), and no element is NaN."""
    lh = gpu
    E, L, H, B = 128, 4096, 32, 4
    announce("flash full config B=4 H=32 S=4096 D=128")
    Q, K, V = attn_inputs(lh, E, L, H, B)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    lh.flash_attn_fwd(O, Q, K, V, causal=True)
    lh.synchronize()
    rng = np.random.default_rng(0)
    rows = np.unique(np.concatenate([[0, 1, 63, 64, 127, 128, 2047, 4095], rng.integers(0, L, 40)]))
    heads = [(0, 0), (3, 31), (1, 17), (2, 5)]
    check_heads(oracle, Q, K, V, O, 1 / math.sqrt(E), True, heads, rows)
    o = O.to_numpy()
    v = V.to_numpy()
    assert not np.isnan(o).any()
    np.testing.assert_array_equal(o[:, 0, :, :], v[:, 0, :, :])


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("scale", [1.0, 0.6, 0.05])
@pytest.mark.parametrize("L", [300, 512])
def test_flash_d128_scales(gpu, oracle, so_kernel, causal, scale, L):
    """The D = 128 kernel folds scale * log2(e) into Q^T when it is at most 1 (0.6, 0.05:
    P = exp2 of the accumulator, the running maximum entering as a bias k-step) and
    multiplies in fp32 otherwise (1.0: scale * log2(e) = 1.44)."""
    lh = gpu
    E, H, B = 128, 2, 1
    announce(f"flash D=128 scale={scale} S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, H, B, cfg=11)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=scale, causal=causal)
    rows = np.unique(np.concatenate([np.arange(0, L, 3), [L - 1]]))
    check_heads(oracle, Q, K, V, O, scale, causal, [(0, 0), (0, 1)], rows)
    assert not np.isnan(O.to_numpy()).any()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("scale", [0.0, -0.0883883])
@pytest.mark.parametrize("E", [128, 64])
def test_flash_scale_zero_and_negative(gpu, oracle, so_kernel, causal, scale, E):
    """A softmax scale of zero (every visible key weighs the same) or below zero (the
    scores change sign, so the running maximum is taken over negated products): D = 128 and
    D = 64 run on the score/output kernel, whose scale folds into Q^T; against the oracle."""
    lh = gpu
    L, H, B = 256, 2, 1
    announce(f"flash D={E} scale={scale} S={L} causal={causal}")
    Q, K, V = attn_inputs(lh, E, L, H, B, cfg=13)
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=scale, causal=causal)
    rows = np.unique(np.concatenate([np.arange(0, L, 5), [L - 1]]))
    check_heads(oracle, Q, K, V, O, scale, causal, [(0, 0), (0, 1)], rows)
    o = O.to_numpy()
    assert not np.isnan(o).any()
    if scale == 0.0:
        # uniform weights: the first query sees only key 0 (causal) or the mean of all keys
        v = V.to_numpy().astype(np.float64)
        want = v[:, 0, :, :] if causal else v.mean(axis=1)
        np.testing.assert_allclose(o[:, 0, :, :].astype(np.float64), want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("causal", [True, False])
def test_flash_d128_maximum_beyond_fp16(gpu, oracle, so_kernel, causal):
    """Scores whose running maximum (in base-2 units) lies beyond +-60000, where the bias
    k-step cannot carry it in fp16: the wavefront switches to the fp32 path.  Scores are
    exact in fp32 (integers): q0 = k0 = 256 plus small integer parts, so every score is
    65536 + q1 k1 with q1, k1 in 0..3 and the softmax stays well conditioned."""
    lh = gpu
    E, L, H, B = 128, 384, 2, 1
    announce(f"flash D=128 maximum beyond fp16 causal={causal}")
    rng = np.random.default_rng(21)
    q = np.zeros((E, L, H, B), np.float16)
    k = np.zeros((E, L, H, B), np.float16)
    q[0], k[0] = 256, 256
    q[1] = rng.integers(0, 4, (L, H, B))
    k[1] = rng.integers(0, 4, (L, H, B))
    v = rng.standard_normal((E, L, H, B)).astype(np.float16)
    Q, K, V = (lh.HIPDeviceArray.from_numpy(np.asfortranarray(a), "f16") for a in (q, k, v))
    O = lh.HIPDeviceArray("f16", (E, L, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=0.69, causal=causal)
    check_heads(oracle, Q, K, V, O, 0.69, causal, [(0, 0), (0, 1)], np.arange(L))
    assert not np.isnan(O.to_numpy()).any()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("E,L", [(128, 300), (64, 512), (96, 300)])
def test_flash_strided_layouts(gpu, oracle, causal, E, L):
    """Q, K, V in (B, L, H, D) memory order (strides 1, D*H, D, D*H*L) and O with padded rows
    (row stride D + 8): the fast kernel addresses every tensor through its strides."""
    lh = gpu
    H, B = 3, 2
    announce(f"flash strided D={E} S={L} causal={causal}")
    st = (1, E * H, E, E * H * L)
    ost = (1, E + 8, (E + 8) * L, (E + 8) * L * H)
    n = E * H * L * B
    bufs = []
    for t in range(3):
        a = lh.HIPDeviceArray("f16", (n,))
        lh.fill_normal(a, lh_mod.seed(7, t))
        bufs.append(a)
    O = lh.HIPDeviceArray("f16", ((E + 8) * L * H * B,))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd_raw(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, O.ptr, B, H, L, E, st, ost, None, causal)
    q, k, v = (a.to_numpy() for a in bufs)
    o = O.to_numpy()
    rows = np.arange(L)
    for (b, h) in [(0, 0), (1, 2), (0, 1)]:
        ref = oracle.attn_rows(q, k, v, L, E, st, 1 / math.sqrt(E), causal, b, h, rows)
        idx = (np.arange(E)[None, :] * ost[0] + rows[:, None] * ost[1] + h * ost[2] + b * ost[3])
        got = o[idx].astype(np.float64)
        assert oracle.rel_frobenius(got, ref) <= 2e-3, (b, h)
        pad = o[(np.arange(8)[None, :] + E) + rows[:, None] * ost[1] + h * ost[2] + b * ost[3]]
        assert np.all(pad.view(np.uint16) == 0xFFFF), "row padding of O written"


@pytest.mark.parametrize("causal", [True, False])
def test_flash_o_rows_8_byte_aligned(gpu, oracle, so_kernel, causal):
    """O with a row stride of D + 4 elements (rows 8-byte aligned only): the D = 128 kernel
    stores O rows in 8-byte pieces instead of staging whole 16-byte-aligned rows."""
    lh = gpu
    E, L, H, B = 128, 320, 2, 1
    announce(f"flash D=128 O rows 8-byte aligned causal={causal}")
    st = (1, E, E * L, E * L * H)
    ost = (1, E + 4, (E + 4) * L, (E + 4) * L * H)
    Q, K, V = attn_inputs(lh, E, L, H, B, cfg=12)
    O = lh.HIPDeviceArray("f16", ((E + 4) * L * H * B,))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd_raw(Q.ptr, K.ptr, V.ptr, O.ptr, B, H, L, E, st, ost, None, causal)
    q, k, v = (a.to_numpy().ravel(order="F") for a in (Q, K, V))
    o = O.to_numpy()
    rows = np.arange(L)
    for h in range(H):
        ref = oracle.attn_rows(q, k, v, L, E, st, 1 / math.sqrt(E), causal, 0, h, rows)
        idx = np.arange(E)[None, :] + rows[:, None] * ost[1] + h * ost[2]
        assert oracle.rel_frobenius(o[idx].astype(np.float64), ref) <= 2e-3, h
        pad = o[(np.arange(4)[None, :] + E) + rows[:, None] * ost[1] + h * ost[2]]
        assert np.all(pad.view(np.uint16) == 0xFFFF), "row padding of O written"
