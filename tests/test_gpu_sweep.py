"""Seeded random shape sweeps through the C ABI against the oracle.

The hand-picked parity cases in the other modules pin each kernel at the shapes its code
paths were written for; these cases draw shapes, layouts, dtypes, head dimensions and
scales from a fixed seed, so that every dispatcher decision (tile kernel, small-product
kernel, mid-size kernel, staged kernel, generic kernels; full and ragged tiles; the W8A16 column-major,
copied-X, split-K and generic kernels; the attention score/output, ping-pong and generic
kernels, and the unsigned GEMM's and the batched W8A16's forms) meets shapes nobody chose.  Same bars as everywhere: int8 bit-exact, fp16/bf16
GEMM and W8A16 relative Frobenius <= 1e-3, attention <= 2e-3.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import lava_hip as lh_mod
from conftest import announce

pytestmark = pytest.mark.gpu


def _dim(rng, lo, hi, mult_p=0.4, mults=(8, 16, 64, 256)):
    """A size in [lo, hi]: with probability mult_p a multiple of one of `mults` (kernels take
    their fast paths on those), otherwise any value."""
    if rng.random() < mult_p:
        m = int(rng.choice(mults))
        top = hi // m
        if top >= 1:
            return int(m * rng.integers(max(1, -(-lo // m)), top + 1))
    return int(rng.integers(lo, hi + 1))


def _gemm_cases():
    rng = np.random.default_rng(20261202)
    out = []
    for _ in range(96):
        dt = str(rng.choice(["f16", "bf16", "i8"]))
        layout = int(rng.integers(0, 8))
        big = rng.random() < 0.3          # past 256 x 256: the tile or the small kernel (rate rule)
        M = _dim(rng, 1, 700 if big else 300)
        N = _dim(rng, 1, 700 if big else 300)
        K = _dim(rng, 1, 600)
        out.append((dt, layout, M, N, K))
    return out


def _mid_cases():
    """Mid-size products with both operands K-contiguous (A row-major, B column-major; C either
    way): the automatic choice among the 128 x 128 mid-size kernel, the tile kernel and the
    small-product kernel at sizes the other draws do not reach."""
    rng = np.random.default_rng(20261128)
    out = []
    for _ in range(12):
        dt = str(rng.choice(["f16", "bf16", "i8"]))
        layout = int(rng.choice([1, 5]))
        M = _dim(rng, 900, 3000, mults=(16, 64, 128))
        N = _dim(rng, 900, 3000, mults=(16, 64, 128))
        K = 16 * int(rng.integers(4, 129))
        out.append((dt, layout, M, N, K))
    return out


def _mid_mn_cases():
    """Mid-size products with an M/N-contiguous operand (A column-major or B row-major; M and N
    multiples of 16, K any where both operands are M/N-contiguous): the mid-size kernel's
    transposing reads under the automatic choice."""
    rng = np.random.default_rng(20261203)
    out = []
    for _ in range(12):
        dt = str(rng.choice(["f16", "bf16", "i8"]))
        layout = int(rng.choice([0, 2, 3, 4, 6, 7]))
        M = 16 * int(rng.integers(57, 188))
        N = 16 * int(rng.integers(57, 188))
        both_mn = layout in (2, 6)
        K = int(rng.integers(64, 2049)) if both_mn else 16 * int(rng.integers(4, 129))
        out.append((dt, layout, M, N, K))
    return out


@pytest.mark.parametrize("dt,layout,M,N,K", _gemm_cases() + _mid_cases() + _mid_mn_cases())
def test_sweep_gemm(gpu, oracle, dt, layout, M, N, K):
    lh = gpu
    announce(f"sweep gemm {dt} layout={layout} M={M} N={N} K={K}")
    A = lh.HIPDeviceArray(dt, (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray(dt, (K, N), order="C" if layout & 2 else "F")
    seed = M * 1000003 + N * 1009 + K
    if dt == "i8":
        lh.fill_i8(A, lh_mod.seed(31, seed))
        lh.fill_i8(B, lh_mod.seed(32, seed))
    else:
        lh.fill_uniform(A, lh_mod.seed(31, seed), -1.0, 1.0)
        lh.fill_uniform(B, lh_mod.seed(32, seed), -1.0, 1.0)
    acc = "i32" if dt == "i8" else "f32"
    C = lh.HIPDeviceArray(acc, (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    a = A.to_numpy().ravel(order=A.order)
    b = B.to_numpy().ravel(order=B.order)
    # every row, or for the mid-size draws 40 seeded rows and the edges (the oracle's time)
    rows = np.arange(M)
    if M * N * K > 1 << 28:
        rows = np.unique(np.concatenate([np.random.default_rng(seed).integers(0, M, 40), [0, 127, 128, M - 1]]))
    got = C.to_numpy()[rows]
    if dt == "i8":
        np.testing.assert_array_equal(got, oracle.gemm_i8_rows(a, b, N, K, lda, ldb, layout & 3, rows))
    else:
        ref = oracle.gemm_rows(a, dt, b, dt, M, N, K, lda, ldb, layout & 3, rows)
        assert oracle.rel_frobenius(got, ref) <= 1e-3


def _attn_cases():
    rng = np.random.default_rng(4096128)
    dims = [8, 16, 24, 32, 40, 64, 72, 96, 120, 128, 136, 160, 200, 256, 12, 50, 100, 130]
    out = []
    for _ in range(48):
        D = int(rng.choice(dims))
        S = _dim(rng, 1, 1500 if rng.random() < 0.3 else 600, mult_p=0.3, mults=(64, 256))
        H = int(rng.integers(1, 4))
        B = int(rng.integers(1, 3))
        causal = bool(rng.random() < 0.6)
        r = rng.random()
        scale = 0.0 if r < 0.1 else (float(rng.uniform(-0.3, -0.01)) if r < 0.25 else
                                     (float(rng.uniform(0.8, 1.5)) if r < 0.4 else 1.0 / math.sqrt(D)))
        out.append((D, S, H, B, causal, round(scale, 6)))
    return out


@pytest.mark.parametrize("D,S,H,B,causal,scale", _attn_cases())
def test_sweep_attention(gpu, oracle, D, S, H, B, causal, scale):
    lh = gpu
    announce(f"sweep flash D={D} S={S} H={H} B={B} causal={causal} scale={scale}")
    Q, K, V = (lh.HIPDeviceArray("f16", (D, S, H, B)) for _ in range(3))
    for t, a in enumerate((Q, K, V)):
        lh.fill_normal(a, lh_mod.seed(41 + t, D * 7919 + S))
    O = lh.HIPDeviceArray("f16", (D, S, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=scale, causal=causal)
    st = (1, D, D * S, D * S * H)
    q, k, v = (a.to_numpy().ravel(order="F") for a in (Q, K, V))
    o = O.to_numpy()
    assert not np.isnan(o).any()
    rows = np.unique(np.concatenate([np.arange(0, S, 3), [S - 1]]))
    for b in range(B):
        for h in range(H):
            ref = oracle.attn_rows(q, k, v, S, D, st, scale, causal, b, h, rows)
            err = oracle.rel_frobenius(o[:, rows, h, b].T.astype(np.float64), ref)
            assert err <= 2e-3, (b, h, err)


def _w8_cases():
    rng = np.random.default_rng(1614336)
    out = []
    for _ in range(48):
        layout = int(rng.integers(0, 8))
        M = _dim(rng, 1, 40, mult_p=0.4, mults=(8, 16))
        N = _dim(rng, 1, 700, mult_p=0.6, mults=(8, 32, 128))
        K = _dim(rng, 1, 800, mult_p=0.6, mults=(16, 32, 128))
        out.append((layout, M, N, K))
    return out


@pytest.mark.parametrize("layout,M,N,K", _w8_cases())
def test_sweep_w8a16(gpu, oracle, layout, M, N, K):
    lh = gpu
    announce(f"sweep w8a16 layout={layout} M={M} N={N} K={K}")
    X = lh.HIPDeviceArray("f16", (M, K), order="C" if layout & 1 else "F")
    W = lh.HIPDeviceArray("i8", (K, N), order="C" if layout & 2 else "F")
    s = lh.HIPDeviceArray("f16", (N,))
    seed = M * 1000003 + N * 1009 + K
    lh.fill_normal(X, lh_mod.seed(51, seed))
    lh.fill_i8(W, lh_mod.seed(52, seed), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(53, seed), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order="C" if layout & 4 else "F")
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    y1 = Y.to_numpy()
    lh.w8a16(Y, X, W, s)
    np.testing.assert_array_equal(Y.to_numpy(), y1)   # fixed summation order: repeat calls identical
    Xh, Wh = np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy())
    ref = oracle.w8a16_rows(Xh, Wh, s.to_numpy(), N, K, K, N, np.arange(M))
    assert oracle.rel_frobenius(y1, ref) <= 1e-3


def _u8_cases():
    rng = np.random.default_rng(255255)
    out = []
    for _ in range(48):
        layout = int(rng.integers(0, 8))
        big = rng.random() < 0.3
        M = _dim(rng, 1, 700 if big else 300, mults=(16, 64, 256))
        N = _dim(rng, 1, 700 if big else 300, mults=(16, 64, 256))
        K = _dim(rng, 1, 2000 if rng.random() < 0.2 else 600, mults=(16, 64, 512))
        out.append((layout, M, N, K))
    return out


@pytest.mark.parametrize("layout,M,N,K", _u8_cases())
def test_sweep_gemm_u8(gpu, oracle, layout, M, N, K):
    """Unsigned bytes: every kernel choice (the tile and small kernels' flipped-byte forms, split
    K, the one-thread-per-element kernel) on drawn shapes, bit for bit."""
    lh = gpu
    announce(f"sweep gemm u8 layout={layout} M={M} N={N} K={K}")
    A = lh.HIPDeviceArray("u8", (M, K), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray("u8", (K, N), order="C" if layout & 2 else "F")
    seed = M * 1000003 + N * 1009 + K
    lh.fill_i8(A, lh_mod.seed(33, seed))
    lh.fill_i8(B, lh_mod.seed(34, seed))
    C = lh.HIPDeviceArray("u32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    lda = K if layout & 1 else M
    ldb = N if layout & 2 else K
    rows = np.unique(np.concatenate([np.arange(0, M, 3), [M - 1]]))
    ref = oracle.gemm_u8_rows(A.to_numpy().ravel(order=A.order), B.to_numpy().ravel(order=B.order), N, K, lda, ldb,
                              layout & 3, rows)
    np.testing.assert_array_equal(C.to_numpy()[rows], ref)


def _w8_batch_cases():
    rng = np.random.default_rng(16300)
    out = []
    for _ in range(16):
        layout = int(rng.integers(0, 8))
        M = int(rng.integers(17, 301))
        N = _dim(rng, 8, 2048, mult_p=0.7, mults=(8, 32, 128))
        K = _dim(rng, 16, 2048, mult_p=0.7, mults=(16, 32, 128))
        out.append((layout, M, N, K))
    return out


@pytest.mark.parametrize("layout,M,N,K", _w8_batch_cases())
def test_sweep_w8a16_batch(gpu, oracle, layout, M, N, K):
    """Batches of 17 to 300 rows (2 or 4 row blocks per workgroup for column-major W, several
    row groups, the row-major copy of X) on drawn shapes; sampled rows against the oracle."""
    lh = gpu
    announce(f"sweep w8a16 batch layout={layout} M={M} N={N} K={K}")
    X = lh.HIPDeviceArray("f16", (M, K), order="C" if layout & 1 else "F")
    W = lh.HIPDeviceArray("i8", (K, N), order="C" if layout & 2 else "F")
    s = lh.HIPDeviceArray("f16", (N,))
    seed = M * 1000003 + N * 1009 + K
    lh.fill_normal(X, lh_mod.seed(54, seed))
    lh.fill_i8(W, lh_mod.seed(55, seed), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(56, seed), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order="C" if layout & 4 else "F")
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    rows = np.unique(np.concatenate([np.arange(0, M, 5), [M - 1]]))
    Xh, Wh = np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy())
    ref = oracle.w8a16_rows(Xh, Wh, s.to_numpy(), N, K, K, N, rows)
    assert oracle.rel_frobenius(Y.to_numpy()[rows], ref) <= 1e-3


# ---- larger shapes: multi-round grids, XCD orders, K splits; sampled rows against the oracle
# and, for the GEMM, every element through sum_ij C_ij = (colsum A) . (rowsum B)
def _gemm_large_cases():
    rng = np.random.default_rng(8192256)
    out = []
    for _ in range(12):
        dt = str(rng.choice(["f16", "bf16", "i8"]))
        layout = int(rng.integers(0, 8))
        M = _dim(rng, 900, 3000, mult_p=0.6, mults=(8, 256))
        N = _dim(rng, 900, 3000, mult_p=0.6, mults=(8, 256))
        K = _dim(rng, 256, 3000, mult_p=0.7, mults=(8, 64, 256))
        out.append((dt, layout, M, N, K))
    return out


@pytest.mark.parametrize("dt,layout,M,N,K", _gemm_large_cases())
def test_sweep_gemm_large(gpu, oracle, dt, layout, M, N, K):
    from test_gpu_gemm import check_rows, full_checksum, make_inputs
    lh = gpu
    announce(f"sweep gemm large {dt} layout={layout} M={M} N={N} K={K}")
    A, B = make_inputs(gpu, dt, M, N, K, layout, lh_mod.seed(61, M + N), lh_mod.seed(62, K))
    C = lh.HIPDeviceArray("i32" if dt == "i8" else "f32", (M, N), order="C" if layout & 4 else "F")
    C.fill_bytes(0xFF)
    lh.gemm(C, A, B)
    rng = np.random.default_rng(M * 31 + N * 17 + K)
    rows = np.unique(np.concatenate([[0, 255, 256, M - 1], rng.integers(0, M, 12)]))
    check_rows(oracle, dt, A, B, C, rows, layout)
    lhs, rhs = full_checksum(C, A, B, dt)
    if dt == "i8":
        assert lhs == rhs
    else:
        assert abs(lhs - rhs) <= 1e-3 * (abs(rhs) + math.sqrt(M * N * K))


def _attn_large_cases():
    rng = np.random.default_rng(40964096)
    out = []
    for D in (64, 96, 128, 128, 128, 200, 256, 48):
        S = _dim(rng, 1000, 4096, mult_p=0.5, mults=(64, 256))
        H = int(rng.integers(1, 9))
        B = int(rng.integers(1, 4))
        causal = bool(rng.random() < 0.75)
        scale = 1.0 / math.sqrt(D) if rng.random() < 0.7 else round(float(rng.uniform(0.02, 0.3)), 6)
        out.append((D, S, H, B, causal, scale))
    return out


@pytest.mark.parametrize("D,S,H,B,causal,scale", _attn_large_cases())
def test_sweep_attention_large(gpu, oracle, D, S, H, B, causal, scale):
    lh = gpu
    announce(f"sweep flash large D={D} S={S} H={H} B={B} causal={causal} scale={scale}")
    Q, K, V = (lh.HIPDeviceArray("f16", (D, S, H, B)) for _ in range(3))
    for t, a in enumerate((Q, K, V)):
        lh.fill_normal(a, lh_mod.seed(71 + t, D * 7919 + S))
    O = lh.HIPDeviceArray("f16", (D, S, H, B))
    O.fill_bytes(0xFF)
    lh.flash_attn_fwd(O, Q, K, V, scale=scale, causal=causal)
    st = (1, D, D * S, D * S * H)
    q, k, v = (a.to_numpy().ravel(order="F") for a in (Q, K, V))
    o = O.to_numpy()
    assert not np.isnan(o).any()
    rng = np.random.default_rng(S * 13 + D)
    rows = np.unique(np.concatenate([[0, 63, 64, 255, 256, S - 1], rng.integers(0, S, 40)]))
    heads = {(0, 0), (B - 1, H - 1), (int(rng.integers(0, B)), int(rng.integers(0, H)))}
    for b, h in sorted(heads):
        ref = oracle.attn_rows(q, k, v, S, D, st, scale, causal, b, h, rows)
        err = oracle.rel_frobenius(o[:, rows, h, b].T.astype(np.float64), ref)
        assert err <= 2e-3, (b, h, err)


def _w8_large_cases():
    rng = np.random.default_rng(1614336 * 2)
    out = []
    for _ in range(10):
        layout = int(rng.integers(0, 8))
        M = int(rng.choice([1, 5, 8, 16, 33, 64]))
        N = _dim(rng, 900, 20000, mult_p=0.7, mults=(8, 32, 128))
        K = _dim(rng, 512, 8192, mult_p=0.8, mults=(16, 32, 128))
        out.append((layout, M, N, K))
    return out


@pytest.mark.parametrize("layout,M,N,K", _w8_large_cases())
def test_sweep_w8a16_large(gpu, oracle, layout, M, N, K):
    lh = gpu
    announce(f"sweep w8a16 large layout={layout} M={M} N={N} K={K}")
    X = lh.HIPDeviceArray("f16", (M, K), order="C" if layout & 1 else "F")
    W = lh.HIPDeviceArray("i8", (K, N), order="C" if layout & 2 else "F")
    s = lh.HIPDeviceArray("f16", (N,))
    lh.fill_normal(X, lh_mod.seed(81, M + K))
    lh.fill_i8(W, lh_mod.seed(82, N + K), symmetric=True)
    lh.fill_uniform(s, lh_mod.seed(83, N), 0.001, 0.02)
    Y = lh.HIPDeviceArray("f32", (M, N), order="C" if layout & 4 else "F")
    Y.fill_bytes(0xFF)
    lh.w8a16(Y, X, W, s)
    y = Y.to_numpy()
    assert not np.isnan(y).any()
    rows = np.unique(np.array([0, M // 2, M - 1]))
    Xh, Wh = np.ascontiguousarray(X.to_numpy()), np.ascontiguousarray(W.to_numpy())
    ref = oracle.w8a16_rows(Xh, Wh, s.to_numpy(), N, K, K, N, rows)
    assert oracle.rel_frobenius(np.ascontiguousarray(y[rows]), ref) <= 1e-3
