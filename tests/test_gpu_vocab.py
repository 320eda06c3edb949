"""Tile-level vocabulary on the GPU, element by element against the oracle:
muladd on 16x16x16 tiles (f16, signed i8, unsigned u8; every layout; 1-based
offsets), the per-element callback (pins the accumulator lane map), the
matrix-operand callback, reduce smears, RNE convert, dot4x8, and the device
input generator.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.npz"


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN))


def dev(lh, a, dtype=None, order="F"):
    return lh.HIPDeviceArray.from_numpy(np.asarray(a), dtype=dtype, order=order)


def flat(lh, a, dtype):
    """1-D device copy of a flat host array."""
    a = np.ascontiguousarray(a).ravel()
    return lh.HIPDeviceArray.from_numpy(a, dtype=dtype)


def test_muladd_i8_golden_tile(gpu, golden):
    lh = gpu
    announce("muladd_16x16x16 i8 golden (l%7, l%5)")
    a = flat(lh, golden["i8_a"].ravel(order="F"), "i8")
    b = flat(lh, golden["i8_b"].ravel(order="F"), "i8")
    c = flat(lh, np.zeros(256, np.int32), "i32")
    d = flat(lh, np.zeros(256, np.int32), "i32")
    lh.coopmat_muladd_16x16x16("i8", "i32", a.ptr, 1, 16, b.ptr, 1, 16, c.ptr, 1, 16, d.ptr, 1, 16, layout=0)
    got = d.to_numpy().reshape(16, 16, order="F")
    np.testing.assert_array_equal(got, golden["i8_c"])
    # signed extremes: -128 * -128 accumulates 16 * 16384 per element
    m = flat(lh, np.full(256, -128, np.int8), "i8")
    lh.coopmat_muladd_16x16x16("i8", "i32", m.ptr, 1, 16, m.ptr, 1, 16, c.ptr, 1, 16, d.ptr, 1, 16)
    np.testing.assert_array_equal(d.to_numpy().reshape(16, 16, order="F"), golden["i8_min_c"])


@pytest.mark.parametrize("dt", ["f32", "f64"])
def test_muladd_wide_identity_pins_layouts(gpu, dt):
    """fp32 / fp64 tiles: A . I + C and I . B + C are exact (every product is by 1 or 0), so they
    pin A's and B's lane layouts independently, bit for bit: a transposed operand read would give
    the transpose, a wrong k slot a zero column.  A non-symmetric M (16 r + c) is used for both."""
    lh = gpu
    announce(f"muladd_16x16x16 {dt} identity products")
    ft = np.float32 if dt == "f32" else np.float64
    m = (16 * np.arange(16)[:, None] + np.arange(16)[None, :]).astype(ft)   # m[r][c] = 16 r + c
    eye = np.eye(16, dtype=ft)
    c = (np.arange(256).reshape(16, 16) * 0.5).astype(ft)
    for a, b, want in ((m, eye, m + c), (eye, m, m + c)):
        da, db, dc = flat(lh, a.ravel(order="F"), dt), flat(lh, b.ravel(order="F"), dt), flat(lh, c.ravel(order="F"), dt)
        dd = flat(lh, np.zeros(256, ft), dt)
        lh.coopmat_muladd_16x16x16(dt, dt, da.ptr, 1, 16, db.ptr, 1, 16, dc.ptr, 1, 16, dd.ptr, 1, 16, layout=0)
        np.testing.assert_array_equal(dd.to_numpy().reshape(16, 16, order="F"), want)


def test_muladd_u8_is_unsigned(gpu, golden):
    lh = gpu
    announce("muladd_16x16x16 u8")
    a = flat(lh, golden["i8_a"].ravel(order="F").astype(np.uint8), "u8")
    b = flat(lh, golden["i8_b"].ravel(order="F").astype(np.uint8), "u8")
    c = flat(lh, np.zeros(256, np.uint32), "u32")
    d = flat(lh, np.zeros(256, np.uint32), "u32")
    lh.coopmat_muladd_16x16x16("u8", "u32", a.ptr, 1, 16, b.ptr, 1, 16, c.ptr, 1, 16, d.ptr, 1, 16)
    np.testing.assert_array_equal(d.to_numpy().reshape(16, 16, order="F"), golden["i8_c"].astype(np.uint32))
    big = flat(lh, np.full(256, 200, np.uint8), "u8")
    lh.coopmat_muladd_16x16x16("u8", "u32", big.ptr, 1, 16, big.ptr, 1, 16, c.ptr, 1, 16, d.ptr, 1, 16)
    assert np.all(d.to_numpy() == 16 * 200 * 200)


@pytest.mark.parametrize("layout", range(16))
@pytest.mark.parametrize("ab,acc", [("f16", "f32"), ("i8", "i32"), ("u8", "u32"), ("f32", "f32"), ("f64", "f64")])
def test_muladd_layouts_offsets_strides(gpu, oracle, layout, ab, acc):
    """Tiles read at 1-based offsets inside larger arrays with padded strides, in
    every row/column-major combination of A, B, C, D, several tiles per call."""
    lh = gpu
    announce(f"muladd_16x16x16 {ab}->{acc} layout={layout}")
    rng = np.random.default_rng(layout)
    ntiles, stride, off = 3, 24, 5
    step = stride * 16 + 7
    total = off + step * ntiles + stride * 16
    if ab in ("f16", "f32", "f64"):
        ft = {"f16": np.float16, "f32": np.float32, "f64": np.float64}[ab]
        A = rng.uniform(-1, 1, total).astype(ft)
        B = rng.uniform(-1, 1, total).astype(ft)
        outdt = np.float64 if ab == "f64" else np.float32
        Cin = rng.uniform(-1, 1, total).astype(outdt)
    elif ab == "i8":
        A = rng.integers(-128, 128, total).astype(np.int8)
        B = rng.integers(-128, 128, total).astype(np.int8)
        Cin = rng.integers(-1000, 1000, total).astype(np.int32)
        outdt = np.int32
    else:
        A = rng.integers(0, 256, total).astype(np.uint8)
        B = rng.integers(0, 256, total).astype(np.uint8)
        Cin = rng.integers(0, 1000, total).astype(np.uint32)
        outdt = np.uint32
    dA, dB, dC = flat(lh, A, ab), flat(lh, B, ab), flat(lh, Cin, acc)
    dD = flat(lh, np.zeros(total, outdt), acc)
    lh.coopmat_muladd_16x16x16(ab, acc, dA.ptr, off, stride, dB.ptr, off + 1, stride, dC.ptr, off + 2, stride,
                               dD.ptr, off + 3, stride, layout=layout, ntiles=ntiles, tile_step=step)
    D = dD.to_numpy()

    def tile(buf, base, rowmajor):
        idx = np.arange(16)
        r, c = np.meshgrid(idx, idx, indexing="ij")
        lin = base + (r * stride + c if rowmajor else c * stride + r)
        return buf[lin]

    for t in range(ntiles):
        a = tile(A, off - 1 + t * step, layout & 1)
        b = tile(B, off + t * step, layout & 2)
        c = tile(Cin, off + 1 + t * step, layout & 4)
        d = tile(D, off + 2 + t * step, layout & 8)
        if ab in ("f16", "f32"):
            ref = a.astype(np.float64) @ b.astype(np.float64) + c.astype(np.float64)
            np.testing.assert_allclose(d, ref, rtol=1e-5, atol=1e-5)
        elif ab == "f64":
            ref = a @ b + c
            np.testing.assert_allclose(d, ref, rtol=1e-13, atol=1e-13)
        else:
            ref = (a.astype(np.int64) @ b.astype(np.int64) + c.astype(np.int64)).astype(outdt)
            np.testing.assert_array_equal(d, ref)


@pytest.mark.parametrize("tile", [16, 32])
def test_perelement_rowcol_pins_lane_map(gpu, golden, tile):
    lh = gpu
    announce(f"perelement rowcol tile={tile}")
    m = golden[f"pe_in_{tile}"]
    ntiles = 3
    host = np.concatenate([(m + k).ravel(order="F") for k in range(ntiles)]).astype(np.float32)
    din = flat(lh, host, "f32")
    dout = flat(lh, np.zeros_like(host), "f32")
    lh.coopmat_perelement_rowcol(din.ptr, dout.ptr, tile, ntiles)
    out = dout.to_numpy()
    for k in range(ntiles):
        got = out[k * tile * tile:(k + 1) * tile * tile].reshape(tile, tile, order="F")
        r = np.arange(tile, dtype=np.float32)[:, None]
        c = np.arange(tile, dtype=np.float32)[None, :]
        ref = ((m + k).astype(np.float32) * (r + np.float32(1)) + c).astype(np.float32)
        np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(out[:tile * tile].reshape(tile, tile, order="F"), golden[f"pe_out_{tile}"])


@pytest.mark.parametrize("tile", [16, 32])
def test_perelement_pair(gpu, oracle, tile):
    lh = gpu
    announce(f"perelement pair tile={tile}")
    rng = np.random.default_rng(tile)
    m = rng.standard_normal((tile, tile)).astype(np.float32)
    o = rng.standard_normal((tile, tile)).astype(np.float32)
    dm, do = flat(lh, m.ravel(order="F"), "f32"), flat(lh, o.ravel(order="F"), "f32")
    dout = flat(lh, np.zeros(tile * tile, np.float32), "f32")
    lh.coopmat_perelement_pair(dm.ptr, do.ptr, dout.ptr, tile, 1)
    np.testing.assert_array_equal(dout.to_numpy().reshape(tile, tile, order="F"), oracle.perelement_pair(m, o))


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("mask", [1, 2, 3])
@pytest.mark.parametrize("combine", ["add", "max", "min"])
def test_reduce_smears(gpu, oracle, tile, mask, combine):
    lh = gpu
    announce(f"reduce tile={tile} mask={mask} {combine}")
    rng = np.random.default_rng(mask * 10 + tile)
    # small integers keep every fp32 sum exact whatever the combining order
    m = rng.integers(-50, 50, (tile, tile)).astype(np.float32)
    din = flat(lh, m.ravel(order="F"), "f32")
    dout = flat(lh, np.zeros(tile * tile, np.float32), "f32")
    lh.coopmat_reduce(din.ptr, dout.ptr, tile, mask, combine, 1)
    got = dout.to_numpy().reshape(tile, tile, order="F")
    np.testing.assert_array_equal(got, oracle.reduce_smear(m, mask, combine).astype(np.float32))


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("mask,dst", [(1, (None, 16)), (1, (None, 64)), (2, (32, None)), (2, (64, None)),
                                      (3, (16, 64)), (3, (64, 32)), (4, "half")])
@pytest.mark.parametrize("combine", ["add", "max", "min"])
def test_reduce_into_other_extent(gpu, oracle, tile, mask, dst, combine):
    """coopmat_reduce into a destination of another extent (Row keeps the rows, Column the
    columns, RowAndColumn any extent; the value smeared over the destination) and the TwoByTwo
    block reduce into tile/2 x tile/2, against the oracle, bit for bit (small integers: every
    fp32 sum exact).  Two tiles per call, each with its own values."""
    lh = gpu
    if dst == "half":
        rd = cd = tile // 2
    else:
        rd = tile if dst[0] is None else dst[0]
        cd = tile if dst[1] is None else dst[1]
    announce(f"reduce_into tile={tile} mask={mask} dst={rd}x{cd} {combine}")
    rng = np.random.default_rng(mask * 100 + tile + rd + cd)
    ms = [rng.integers(-50, 50, (tile, tile)).astype(np.float32) for _ in range(2)]
    din = flat(lh, np.concatenate([m.ravel(order="F") for m in ms]), "f32")
    dout = flat(lh, np.full(2 * rd * cd, np.nan, np.float32), "f32")
    lh.coopmat_reduce_into(din.ptr, dout.ptr, tile, rd, cd, mask, combine, 2)
    got = dout.to_numpy()
    for t, m in enumerate(ms):
        g = got[t * rd * cd:(t + 1) * rd * cd].reshape(rd, cd, order="F")
        want = oracle.reduce_2x2(m, combine) if mask == 4 else oracle.reduce_into(m, mask, combine, rd, cd)
        np.testing.assert_array_equal(g, want.astype(np.float32))


def test_reduce_into_shape_errors(gpu):
    lh = gpu
    announce("reduce_into shape errors")
    for tile, rd, cd, mask in [(16, 32, 16, 1), (16, 16, 32, 2), (16, 16, 16, 4), (32, 16, 128, 3), (16, 16, 8, 1)]:
        with pytest.raises(lh.InvalidArgument):
            lh.coopmat_reduce_into(8, 8, tile, rd, cd, mask, "add", 1)
    with pytest.raises(lh.Unsupported):
        lh.coopmat_reduce(8, 8, 16, 4, "add", 1)   # the same-shape form has no TwoByTwo


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_convert_rne(gpu, oracle, golden, dt):
    lh = gpu
    announce(f"convert f32->{dt}")
    rng = np.random.default_rng(4)
    edges = golden["narrow_in"].astype(np.float32)
    bits = rng.integers(0, 2 ** 32, 1 << 18, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([edges, bits.view(np.float32), np.zeros(256 - (edges.size + bits.size) % 256, np.float32)])
    x[np.isnan(x)] = 1.0
    din = flat(lh, x, "f32")
    dout = flat(lh, np.zeros(x.size, np.uint16), "bf16")
    lh.coopmat_convert(din.ptr, dout.ptr, dt, x.size)
    got = dout.to_numpy()
    ref = oracle.f32_to_f16_bits(x) if dt == "f16" else oracle.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(got, ref)


def test_dot4x8(gpu, oracle, golden):
    lh = gpu
    announce("dot4x8")
    rng = np.random.default_rng(5)
    a = np.concatenate([golden["dot_a"], rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32)])
    b = np.concatenate([golden["dot_b"], rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32)])
    da, db = flat(lh, a, "u32"), flat(lh, b, "u32")
    dy = flat(lh, np.zeros(a.size, np.int32), "i32")
    lh.dot4x8(da.ptr, db.ptr, dy.ptr, a.size)
    np.testing.assert_array_equal(dy.to_numpy(), oracle.dot4x8(a, b))


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_device_generator_matches_oracle(gpu, oracle, dt):
    lh = gpu
    announce(f"fill {dt}")
    n = (1 << 20) + 3
    d = lh.HIPDeviceArray(dt, (n,))
    lh.fill_uniform(d, 0x4C415641, -1.0, 1.0)
    np.testing.assert_array_equal(d.to_numpy(), oracle.fill_uniform(n, dt, 0x4C415641, -1.0, 1.0))
    lh.fill_uniform(d, 99, 0.001, 0.02)
    np.testing.assert_array_equal(d.to_numpy(), oracle.fill_uniform(n, dt, 99, 0.001, 0.02))
    lh.fill_normal(d, 123)
    got, ref = d.to_numpy(), oracle.fill_normal(n, dt, 123)
    # libm and the device math library may differ in the last bit of log/cos; a
    # differing element must then be one unit of the storage type apart
    diff = np.flatnonzero(got.view(np.uint16 if dt != "f32" else np.uint32) != ref.view(np.uint16 if dt != "f32" else np.uint32))
    assert diff.size <= 16, diff[:20]
    i8 = lh.HIPDeviceArray("i8", (n,))
    for sym in (False, True):
        lh.fill_i8(i8, 7, sym)
        np.testing.assert_array_equal(i8.to_numpy(), oracle.fill_i8(n, 7, sym))
