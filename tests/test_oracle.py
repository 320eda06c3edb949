"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is compared with a source that does not share its code:
numpy / torch library routines (matmul, float16 and bfloat16 casts), closed
forms (identity, one-hot, constant inputs), brute force on tiny inputs, and the
golden vectors of tests/golden/known_answers.npz (numpy-computed from the
reference's own known-answer cases).  Planted mistakes (a transposed operand, a
dropped scale, a shifted mask) are shown to fail these checks.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.npz"

LAYOUTS = list(range(4))   # bit0 A row-major, bit1 B row-major


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN))


def _store(mat: np.ndarray, rowmajor: bool) -> tuple[np.ndarray, int]:
    """Flat storage of a matrix in the given order and its leading dimension."""
    if rowmajor:
        return np.ascontiguousarray(mat).ravel(), mat.shape[1]
    return np.asfortranarray(mat).ravel(order="F"), mat.shape[0]


# ---------------------------------------------------------------- generator
def test_rng_matches_splitmix64_reference_stream(oracle):
    # seed 0 makes the counter stream exactly splitmix64 started from state 0, whose
    # published first outputs are these
    assert oracle.rng_u64(0, 0) == 0xE220A8397B1DCDAF
    assert oracle.rng_u64(0, 1) == 0x6E789E6AA1B965F4
    assert oracle.rng_u64(0, 2) == 0x06C45D188009454F


def test_rng_matches_independent_numpy_finaliser(oracle):
    seed = 0x4C415641
    i = np.arange(1000, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) * np.uint64(0xD1B54A32D192ED03) + (i + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    got = np.array([oracle.rng_u64(seed, int(k)) for k in i], dtype=np.uint64)
    np.testing.assert_array_equal(got, z)


def test_uniform_definition(oracle):
    seed, n = 77, 4096
    v = oracle.fill_uniform(n, "f32", seed, -1.0, 1.0)
    k = np.array([oracle.rng_u64(seed, i) >> 40 for i in range(n)], dtype=np.float64)
    np.testing.assert_array_equal(v, (-1.0 + 2.0 * k * 2.0 ** -24).astype(np.float32))
    assert v.min() >= -1 and v.max() < 1
    h = oracle.fill_uniform(n, "f16", seed, -1.0, 1.0)
    np.testing.assert_array_equal(h, v.astype(np.float16))
    s = oracle.fill_uniform(n, "f16", seed, 0.001, 0.02)
    assert s.min() >= np.float16(0.001) and s.max() <= np.float16(0.02)


def test_normal_and_int8_statistics(oracle):
    n = 1 << 20
    x = oracle.fill_normal(n, "f32", 5).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1) < 5e-3
    z = oracle.rng_u64(5, 17)
    u1 = ((z >> 32) + 0.5) * 2.0 ** -32
    u2 = ((z & 0xFFFFFFFF) + 0.5) * 2.0 ** -32
    import math
    assert x[17] == np.float32(math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2))
    a = oracle.fill_i8(n, 9, symmetric=False)
    assert a.min() == -128 and a.max() == 127
    s = oracle.fill_i8(n, 9, symmetric=True)
    assert s.min() == -127 and s.max() == 127
    assert abs(a.astype(np.float64).mean() + 0.5) < 0.2


# ---------------------------------------------------------------- narrowing
def test_f16_narrowing_golden_edges(oracle, golden):
    np.testing.assert_array_equal(oracle.f32_to_f16_bits(golden["narrow_in"]), golden["narrow_f16_bits"])


def test_f16_narrowing_matches_numpy_sweep(oracle):
    rng = np.random.default_rng(1)
    # every mantissa of the exponents around the half range, plus random bit patterns
    exps = np.arange(96, 146, dtype=np.uint32)   # 2^-31 .. 2^18
    mant = rng.integers(0, 1 << 23, size=4096, dtype=np.uint32)
    bits = ((exps[:, None] << 23) | mant[None, :]).ravel()
    bits = np.concatenate([bits, bits | 0x80000000, rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)])
    x = bits.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16_bits(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_bf16_narrowing_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    bits[:6] = [0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7FFFFF, 0x00000001, 0x80000000]
    x = bits.view(np.float32)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle.f32_to_bf16_bits(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], ref[~nan])


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_gemm_rows_matches_numpy(oracle, layout, dt):
    rng = np.random.default_rng(layout)
    M, N, K = 37, 29, 53
    A = oracle.fill_uniform(M * K, dt, 11 + layout, -1, 1).reshape(M, K)
    B = oracle.fill_uniform(K * N, dt, 12 + layout, -1, 1).reshape(K, N)
    Ad, Bd = oracle.decode(A, dt), oracle.decode(B, dt)
    As, lda = _store(A, bool(layout & 1))
    Bs, ldb = _store(B, bool(layout & 2))
    rows = rng.permutation(M)[:10]
    got = oracle.gemm_rows(As, dt, Bs, dt, M, N, K, lda, ldb, layout, rows)
    np.testing.assert_allclose(got, (Ad @ Bd)[rows], rtol=0, atol=1e-12)


def test_gemm_golden_and_closed_forms(oracle, golden):
    A, B = golden["gemm_a"], golden["gemm_b"]
    M, K = A.shape
    N = B.shape[1]
    got = oracle.gemm_rows(A.ravel(), "f16", B.ravel(), "f16", M, N, K, K, N, 3, np.arange(M))
    np.testing.assert_allclose(got, golden["gemm_c"], rtol=0, atol=1e-12)
    # identity: I * B = B exactly
    I = np.eye(K, dtype=np.float16)
    got = oracle.gemm_rows(I.ravel(), "f16", B.ravel(), "f16", K, N, K, K, N, 3, np.arange(K))
    np.testing.assert_array_equal(got, B.astype(np.float64))
    # planted mistake: reading A with the wrong layout must not reproduce the product
    bad = oracle.gemm_rows(A.ravel(), "f16", B.ravel(), "f16", M, N, K, K, N, 2, np.arange(M))
    assert oracle.rel_frobenius(bad, golden["gemm_c"]) > 0.1


def test_gemm_f32acc_close_to_fp64(oracle):
    M, N, K = 16, 64, 512
    A = oracle.fill_uniform(M * K, "bf16", 3, -1, 1)
    B = oracle.fill_uniform(K * N, "bf16", 4, -1, 1)
    ref = oracle.gemm_rows(A, "bf16", B, "bf16", M, N, K, K, K, 1, np.arange(M))
    got = oracle.gemm_f32acc(A, "bf16", B, "bf16", N, K, K, K, 1, M)
    assert oracle.rel_frobenius(got, ref) < 1e-5


def test_gemm_i8_exact_vs_numpy_and_golden(oracle, golden):
    a, b = golden["i8_a"], golden["i8_b"]
    # column-major storage of both (layout 0)
    got = oracle.gemm_i8_rows(a.ravel(order="F"), b.ravel(order="F"), 16, 16, 16, 16, 0, np.arange(16))
    np.testing.assert_array_equal(got, golden["i8_c"])
    full = np.full((16, 16), -128, dtype=np.int8)
    got = oracle.gemm_i8_rows(full.ravel(), full.ravel(), 16, 16, 16, 16, 3, np.arange(16))
    np.testing.assert_array_equal(got, golden["i8_min_c"])
    M, N, K = 33, 47, 300
    A = oracle.fill_i8(M * K, 21).reshape(M, K)
    B = oracle.fill_i8(K * N, 22).reshape(K, N)
    got = oracle.gemm_i8_rows(A.ravel(), np.asfortranarray(B).ravel(order="F"), N, K, K, K, 1, np.arange(M))
    np.testing.assert_array_equal(got, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.int32))


def test_gemm_u8_exact_is_unsigned(oracle, golden):
    a = golden["i8_a"].astype(np.uint8)
    b = golden["i8_b"].astype(np.uint8)
    got = oracle.gemm_u8_rows(a.ravel(order="F"), b.ravel(order="F"), 16, 16, 16, 16, 0, np.arange(16))
    np.testing.assert_array_equal(got, golden["i8_c"].astype(np.uint32))
    big = np.full((16, 16), 200, dtype=np.uint8)
    got = oracle.gemm_u8_rows(big.ravel(), big.ravel(), 16, 16, 16, 16, 3, np.arange(16))
    assert np.all(got == 16 * 200 * 200)   # signed reading would give 16 * 56 * 56


def test_w8a16_matches_numpy(oracle):
    M, N, K = 16, 96, 256
    X = oracle.fill_normal(M * K, "f16", 31).reshape(M, K)
    W = oracle.fill_i8(K * N, 32, symmetric=True).reshape(K, N)
    s = oracle.fill_uniform(N, "f16", 33, 0.001, 0.02)
    got = oracle.w8a16_rows(X, W, s, N, K, K, N, np.arange(M))
    ref = (X.astype(np.float64) @ W.astype(np.float64)) * s.astype(np.float64)[None, :]
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # planted mistake: dropping the scale fails
    assert oracle.rel_frobenius(X.astype(np.float64) @ W.astype(np.float64), ref) > 0.5


# ---------------------------------------------------------------- attention
def _attn_numpy(Q, K, V, scale, causal):
    E, L, H, B = Q.shape
    O = np.zeros((E, L, H, B))
    for b in range(B):
        for h in range(H):
            q, k, v = (x[:, :, h, b].T.astype(np.float64) for x in (Q, K, V))
            s = q @ k.T * scale
            if causal:
                s[np.triu_indices(L, 1)] = -np.inf
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            O[:, :, h, b] = (p @ v).T
    return O


def _attn_oracle(oracle, Q, K, V, scale, causal, b, h, rows):
    E, L, H, B = Q.shape
    st = (1, E, E * L, E * L * H)
    return oracle.attn_rows(Q.ravel(order="F"), K.ravel(order="F"), V.ravel(order="F"), L, E, st, scale, causal, b, h,
                            rows)


def test_attn_golden(oracle, golden):
    Q, K, V = golden["attn_q"], golden["attn_k"], golden["attn_v"]
    E, L, H, _ = Q.shape
    for h in range(H):
        got = _attn_oracle(oracle, Q, K, V, 1 / np.sqrt(E), True, 0, h, np.arange(L))
        np.testing.assert_allclose(got, golden["attn_o"][:, :, h, 0].T, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_attn_matches_numpy(oracle, causal):
    E, L, H, B = 32, 48, 2, 2
    g = np.random.default_rng(7)
    Q, K, V = (g.standard_normal((E, L, H, B)).astype(np.float16) for _ in range(3))
    ref = _attn_numpy(Q, K, V, 0.3, causal)
    for b in range(B):
        for h in range(H):
            got = _attn_oracle(oracle, Q, K, V, 0.3, causal, b, h, np.arange(L))
            np.testing.assert_allclose(got, ref[:, :, h, b].T, rtol=1e-10, atol=1e-12)


def test_attn_closed_forms(oracle):
    E, L = 16, 40
    g = np.random.default_rng(8)
    V = g.standard_normal((E, L, 1, 1)).astype(np.float16)
    K = g.standard_normal((E, L, 1, 1)).astype(np.float16)
    Q = np.zeros((E, L, 1, 1), dtype=np.float16)
    # all scores equal -> causal row i is the mean of v_0 .. v_i
    got = _attn_oracle(oracle, Q, K, V, 1.0, True, 0, 0, np.arange(L))
    v = V[:, :, 0, 0].T.astype(np.float64)
    np.testing.assert_allclose(got, np.cumsum(v, axis=0) / np.arange(1, L + 1)[:, None], rtol=1e-12, atol=1e-12)
    # causal row 0 is v_0 whatever q is
    Q2 = g.standard_normal((E, L, 1, 1)).astype(np.float16)
    got = _attn_oracle(oracle, Q2, K, V, 0.25, True, 0, 0, [0])
    np.testing.assert_allclose(got[0], v[0], rtol=0, atol=1e-15)
    # planted mistake: a mask shifted by one key fails the cumulative-mean form
    bad = np.concatenate([v[:1], (np.cumsum(v, axis=0)[1:] - v[1:]) / np.arange(1, L)[:, None]])
    assert np.abs(bad - np.cumsum(v, axis=0) / np.arange(1, L + 1)[:, None]).max() > 1e-3


# ---------------------------------------------------------------- scalar / tile
def test_dot4x8_golden_and_brute_force(oracle, golden):
    np.testing.assert_array_equal(oracle.dot4x8(golden["dot_a"], golden["dot_b"]), golden["dot_y"])
    assert oracle.dot4x8(np.array([0x80808080], np.uint32), np.array([0x80808080], np.uint32))[0] == 65536
    g = np.random.default_rng(3)
    a = g.integers(0, 2 ** 32, size=10000, dtype=np.uint64).astype(np.uint32)
    b = g.integers(0, 2 ** 32, size=10000, dtype=np.uint64).astype(np.uint32)
    ba = a.view(np.uint8).reshape(-1, 4).view(np.int8).astype(np.int64)
    bb = b.view(np.uint8).reshape(-1, 4).view(np.int8).astype(np.int64)
    np.testing.assert_array_equal(oracle.dot4x8(a, b), (ba * bb).sum(axis=1))


def test_perelement_and_reduce_definitions(oracle, golden):
    for t in (16, 32):
        np.testing.assert_array_equal(oracle.perelement_rowcol(golden[f"pe_in_{t}"]), golden[f"pe_out_{t}"])
    m = np.arange(16 * 16, dtype=np.float32).reshape(16, 16)
    r = oracle.reduce_smear(m, 1, "max")
    assert np.all(r == m[:, -1:])            # row max smeared along the row
    c = oracle.reduce_smear(m, 2, "add")
    assert np.all(c == m.sum(axis=0, keepdims=True))
    both = oracle.reduce_smear(m, 3, "min")
    assert np.all(both == 0)
    p = oracle.perelement_pair(m, m.T.copy())
    assert p[2, 5] == max(m[2, 5], m[5, 2]) + 2 - 5


def test_reduce_into_and_two_by_two_definitions(oracle):
    """The reduce into another extent against closed forms of an arange tile (row r of m is
    16 r + [0, 16): its max is 16 r + 15, its sum 256 r + 120), and the TwoByTwo block reduce
    against an independent formulation (a reshape to (R/2, 2, C/2, 2) reduced over the block
    axes); a transposed operand or a swapped block index fails both."""
    m = np.arange(16 * 16, dtype=np.float32).reshape(16, 16)
    r = oracle.reduce_into(m, 1, "max", 16, 64)
    assert r.shape == (16, 64) and np.all(r == (16 * np.arange(16) + 15)[:, None])
    c = oracle.reduce_into(m, 2, "add", 32, 16)
    assert c.shape == (32, 16) and np.all(c == (16 * 120 + 16 * np.arange(16))[None, :])
    s = oracle.reduce_into(m, 3, "min", 64, 32)
    assert s.shape == (64, 32) and np.all(s == 0)
    rng = np.random.default_rng(3)
    x = rng.integers(-100, 100, (32, 32)).astype(np.float32)
    for comb, f in (("add", np.sum), ("max", np.max), ("min", np.min)):
        want = f(x.reshape(16, 2, 16, 2), axis=(1, 3))
        np.testing.assert_array_equal(oracle.reduce_2x2(x, comb), want)
    # a mistake a block reduce can make: pairing rows 2i and 2i+1 of the transposed tile
    assert not np.array_equal(oracle.reduce_2x2(x.T, "max"), oracle.reduce_2x2(x, "max"))


# ---------------------------------------------------------------- GEMM epilogue
def test_gelu_closed_forms(oracle):
    """erf form: gelu(x) = x Phi(x) -- Phi(1) = 0.8413447460685429 (standard normal
    CDF at 1), gelu(0) = 0, gelu(x) -> x and -> 0 far out; the tanh form is the
    published approximation, within 1e-3 of the erf form on [-6, 6]."""
    x = np.array([0.0, 1.0, -1.0, 8.0, -8.0])
    ge = oracle.gelu_erf(x)
    assert ge[0] == 0.0
    assert abs(ge[1] - 0.8413447460685429) < 1e-15
    assert abs(ge[2] - (-1.0 + 0.8413447460685429)) < 1e-15   # gelu(-x) = gelu(x) - x
    assert abs(ge[3] - 8.0) < 1e-12 and abs(ge[4]) < 1e-12
    t = np.linspace(-6, 6, 1201)
    assert np.abs(oracle.gelu_tanh(t) - oracle.gelu_erf(t)).max() < 1e-3
    assert abs(oracle.gelu_tanh(np.array([1.0]))[0] - 0.8411919906082768) < 1e-15


def test_gemm_epilogue_accinit_axes(oracle):
    """bias is one value per row (a stride-0 accumulator load: every column reads the
    same vector), the residual is added elementwise, the activation comes last."""
    c = np.arange(12, dtype=np.float64).reshape(3, 4) - 6.0
    bias = np.array([10.0, -20.0, 0.5])
    res = np.full((3, 4), 0.25)
    d = oracle.gemm_epilogue(c, bias, res, "relu")
    np.testing.assert_array_equal(d, np.maximum(c + bias[:, None] + 0.25, 0.0))
    # planted mistake: a bias broadcast along columns gives a different matrix
    assert not np.array_equal(d, np.maximum(c + np.resize(bias, 4)[None, :] + 0.25, 0.0))
    np.testing.assert_array_equal(oracle.gemm_epilogue(c), c)


def test_round_to_rne(oracle):
    x = np.array([1.0 + 2.0 ** -9, 1.0 + 3 * 2.0 ** -9, 65504.0, 1.0 + 2.0 ** -11])
    assert oracle.round_to(x[:2], "bf16").tolist() == [1.0, 1.0078125]
    assert oracle.round_to(x[2:], "f16").tolist() == [65504.0, 1.0]   # tie to even
    assert oracle.round_to(np.array([0.1]), "f32")[0] == float(np.float32(0.1))


# ---- tensor addressing --------------------------------------------------------------
def _layout(dims, strides=None, off=None, size=None, clamp=1, rank=None):
    rank = rank or len(dims)
    if strides is None:
        strides, s = [0] * rank, 1
        for i in range(rank - 1, -1, -1):
            strides[i] = s
            s *= dims[i]
    return {"rank": rank, "clamp": clamp, "dim": list(dims), "stride": list(strides),
            "off": list(off or [0] * rank), "size": list(size or dims)}


def test_tensor_load_inside_is_submatrix(oracle):
    """A slice inside the tensor is the submatrix, for a packed and a padded (ld 37) tensor."""
    for ld in (30, 37):
        mem = np.arange(20 * ld, dtype=np.float64)
        l = _layout((20, 30), (ld, 1), (3, 5), (16, 16))
        got = oracle.tensor_load(np.zeros((16, 16)), mem, l, -1.0)
        np.testing.assert_array_equal(got, mem.reshape(20, ld)[3:19, 5:21])


@pytest.mark.parametrize("mode,pad", [(1, "constant"), (2, "edge")])
def test_tensor_load_clamp_modes_are_pads(oracle, mode, pad):
    """CONSTANT reads the clamp value outside the tensor, TO_EDGE the nearest element:
    exactly numpy.pad's constant and edge modes, for slices over every edge."""
    mem = np.arange(20 * 30, dtype=np.float64) * 0.5 + 1.0
    t = mem.reshape(20, 30)
    kw = {"constant_values": 7.0} if pad == "constant" else {}
    padded = np.pad(t, 16, mode=pad, **kw)
    for off in [(-3, 20), (10, -7), (-16, -16), (15, 25), (19, 29), (40, 2)]:
        l = _layout((20, 30), (30, 1), off, (16, 16), clamp=mode)
        got = oracle.tensor_load(np.zeros((16, 16)), mem, l, 7.0)
        r, c = off[0] + 16, off[1] + 16
        want = np.full((16, 16), 7.0) if pad == "constant" and r >= padded.shape[0] else None
        if want is None:
            block = padded[max(r, 0):r + 16, max(c, 0):c + 16]
            if block.shape != (16, 16):   # beyond numpy's 16-element pad: extend it by its own rule
                block = np.pad(t, 64, mode=pad, **kw)[r + 48:r + 64, c + 48:c + 64]
            want = block
        np.testing.assert_array_equal(got, want, err_msg=f"off={off} mode={pad}")


def test_tensor_load_transposing_view(oracle):
    """Through the (1, 0) view, matrix (r, c) reads slice (c, r): an 8 x 16 matrix from a
    16 x 8 slice is that slice transposed; without the view the same load differs."""
    mem = np.arange(20 * 30, dtype=np.float64)
    l = _layout((20, 30), (30, 1), (2, 4), (16, 8))
    got = oracle.tensor_load(np.zeros((8, 16)), mem, l, 0.0, transpose=True)
    np.testing.assert_array_equal(got, mem.reshape(20, 30)[2:18, 4:12].T)
    plain = oracle.tensor_load(np.zeros((8, 16)), mem, dict(l, size=[8, 16]), 0.0)
    assert not np.array_equal(plain, got)


def test_tensor_load_undefined_keeps_object_outside_tensor(oracle):
    """UNDEFINED: elements of the slice past the tensor keep the object's value (the
    clamp constant is not read); the elements inside are the submatrix."""
    mem = np.arange(20 * 30, dtype=np.float64)
    obj = np.full((16, 16), -3.0)
    l = _layout((20, 30), (30, 1), (10, 20), (16, 16), clamp=0)
    got = oracle.tensor_load(obj, mem, l, 99.0)
    np.testing.assert_array_equal(got[:10, :10], mem.reshape(20, 30)[10:20, 20:30])
    assert np.all(got[10:, :] == -3.0) and np.all(got[:, 10:] == -3.0)


def test_tensor_load_keeps_object_outside_slice(oracle):
    mem = np.arange(20 * 30, dtype=np.float64)
    obj = np.full((16, 16), -5.0)
    l = _layout((20, 30), (30, 1), (1, 2), (10, 12))
    got = oracle.tensor_load(obj, mem, l, 0.0)
    np.testing.assert_array_equal(got[:10, :12], mem.reshape(20, 30)[1:11, 2:14])
    assert np.all(got[10:, :] == -5.0) and np.all(got[:, 12:] == -5.0)


def test_tensor_load_rank3_outer_block(oracle):
    """A rank-3 slice picks its outer block by offset; an outer offset past the tensor reads
    the clamp value (CONSTANT) or the last block (TO_EDGE)."""
    mem = np.arange(4 * 20 * 30, dtype=np.float64)
    t = mem.reshape(4, 20, 30)
    l = _layout((4, 20, 30), None, (2, 3, 5), (1, 16, 16))
    np.testing.assert_array_equal(oracle.tensor_load(np.zeros((16, 16)), mem, l, 0.0), t[2, 3:19, 5:21])
    out = dict(l, off=[5, 3, 5])
    assert np.all(oracle.tensor_load(np.zeros((16, 16)), mem, out, 9.0) == 9.0)
    np.testing.assert_array_equal(oracle.tensor_load(np.zeros((16, 16)), mem, dict(out, clamp=2), 9.0),
                                  t[3, 3:19, 5:21])


def test_tensor_store_writes_inside_only(oracle):
    """The clamping store writes slice ∩ tensor; through the view, the transpose."""
    dst = np.full(20 * 30, -1.0)
    m = np.arange(256, dtype=np.float64).reshape(16, 16)
    l = _layout((20, 30), (30, 1), (10, 20), (16, 16), clamp=2)   # a store never clamps to the edge
    got = oracle.tensor_store(m, dst, l).reshape(20, 30)
    want = np.full((20, 30), -1.0)
    want[10:20, 20:30] = m[:10, :10]
    np.testing.assert_array_equal(got, want)
    got_t = oracle.tensor_store(m, dst, l, transpose=True).reshape(20, 30)
    want_t = np.full((20, 30), -1.0)
    want_t[10:20, 20:30] = m.T[:10, :10]
    np.testing.assert_array_equal(got_t, want_t)


def test_tensor_clamp_one_gives_row_sums(oracle):
    """The V-padding identity: with V's columns past the tensor read as one, those columns
    of P V are the row sums of P."""
    rng = np.random.default_rng(3)
    P = rng.random((16, 16))
    E = 10
    V = rng.random(16 * E)
    l = _layout((16, E), (E, 1), (0, 0), (16, 16))
    Vp = oracle.tensor_load(np.zeros((16, 16)), V, l, 1.0)
    D = P @ Vp
    np.testing.assert_allclose(D[:, :E], P @ V.reshape(16, E), rtol=1e-14)
    np.testing.assert_allclose(D[:, E:], np.repeat(P.sum(axis=1, keepdims=True), 16 - E, axis=1), rtol=1e-14)


# ---------------------------------------------------------------- tile addressing and per-element scales
def test_load_tile_matches_numpy_reshapes_and_strided_views(oracle):
    rng = np.random.default_rng(3)
    buf = rng.standard_normal(4096).astype(np.float32)
    R, C, off = 16, 32, 7
    # packed: numpy's own F / C reshapes of the contiguous run
    np.testing.assert_array_equal(oracle.load_tile(buf, off, R, False, R, C),
                                  buf[off:off + R * C].reshape(R, C, order="F"))
    np.testing.assert_array_equal(oracle.load_tile(buf, off, C, True, R, C),
                                  buf[off:off + R * C].reshape(R, C))
    # padded strides: numpy's strided view of the same memory
    isz = buf.itemsize
    for s in (R + 3, 40):
        view = np.lib.stride_tricks.as_strided(buf[off:], shape=(R, C), strides=(isz, s * isz))
        np.testing.assert_array_equal(oracle.load_tile(buf, off, s, False, R, C), view)
    view = np.lib.stride_tricks.as_strided(buf[off:], shape=(R, C), strides=(45 * isz, isz))
    np.testing.assert_array_equal(oracle.load_tile(buf, off, 45, True, R, C), view)


def test_load_tile_stride_zero_broadcasts(oracle):
    """Stride 0: every column (column-major) reads the same R-vector -- a per-row factor;
    every row (row-major) reads the same C-vector -- a per-column factor."""
    v = np.arange(100, dtype=np.float32) * 0.5
    np.testing.assert_array_equal(oracle.load_tile(v, 3, 0, False, 16, 16),
                                  np.broadcast_to(v[3:19][:, None], (16, 16)))
    np.testing.assert_array_equal(oracle.load_tile(v, 5, 0, True, 16, 32),
                                  np.broadcast_to(v[5:37][None, :], (16, 32)))
    # a planted transposition (the column-major rule read row-major) fails it
    wrong = oracle.load_tile(v, 3, 0, True, 16, 16)
    assert not np.array_equal(wrong, np.broadcast_to(v[3:19][:, None], (16, 16)))


def test_store_tile_round_trip_and_untouched(oracle):
    rng = np.random.default_rng(4)
    buf = np.zeros(2048, np.float32)
    m = rng.standard_normal((32, 32)).astype(np.float32)
    for rowmajor in (False, True):
        out = oracle.store_tile(buf, 11, 50, rowmajor, m)
        np.testing.assert_array_equal(oracle.load_tile(out, 11, 50, rowmajor, 32, 32), m)
        assert np.count_nonzero(out) == np.count_nonzero(m)   # nothing else written
        assert out[:11].sum() == 0


def test_scale_columns_and_rows_are_diagonal_products(oracle):
    """Per-column scaling is M diag(s); per-row is diag(cs) M: numpy matmul in fp64 of the
    same values (each element one product, so fp32 rounding of it is exact to 1 ulp)."""
    rng = np.random.default_rng(5)
    m = rng.standard_normal((16, 16)).astype(np.float32)
    s = rng.uniform(0.001, 0.02, 64).astype(np.float16)
    got = oracle.scale_columns(m, s, 9)
    ref = m.astype(np.float64) @ np.diag(s[9:25].astype(np.float64))
    np.testing.assert_array_equal(got, ref.astype(np.float32))
    cs = rng.standard_normal(64).astype(np.float32)
    got = oracle.scale_rows(m, cs, 30)
    ref = np.diag(cs[30:46].astype(np.float64)) @ m.astype(np.float64)
    np.testing.assert_array_equal(got, ref.astype(np.float32))
    # a planted row/column swap fails
    assert not np.array_equal(oracle.scale_rows(m, s.astype(np.float32), 9), oracle.scale_columns(m, s, 9))
