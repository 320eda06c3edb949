"""The rest of the tile vocabulary on the GPU, against the oracle:

- convert with a change of use (fp32 Accumulator -> fp16/bf16 MatrixA / MatrixB), and
  the P -> MatrixA step feeding a second product (coopmat_intrinsics.jl:222-247);
- coopmat_mul / coopmat_add, including the stride-0 broadcast factor and `accinit`
  (coopmat_intrinsics.jl:402-464);
- the length / getcomp / setcomp elementwise loop (coopmat_intrinsics.jl:322-400);
- perelement with a pointer and an offset in `extras` (coopmat_intrinsics.jl:569-572);
- the device half of caps(): the hipDeviceProp record, the MFMA table and the
  workgroup-scope table `wggran`, each row run as a workgroup-scope GEMM (caps.jl:54-159).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def flat(lh, a, dtype):
    return lh.HIPDeviceArray.from_numpy(np.ascontiguousarray(a).ravel(), dtype=dtype)


def zeros(lh, n, dtype):
    return flat(lh, np.zeros(n, {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i32": np.int32}[dtype]),
                dtype)


def edge_values(rng, n):
    """fp32 values with narrowing edge cases mixed into normal(0, 1)."""
    x = rng.standard_normal(n).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65520.0, -65520.0, 1e-8, 5.9604645e-08, 2.9802322e-08, 1.0 + 2 ** -11,
                      1.0 + 3 * 2 ** -11, 3.4e38, np.inf, -np.inf], np.float32)
    x[:edges.size] = edges
    return x


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("use", ["MatrixA", "MatrixB", "Accumulator"])
def test_convert_use_is_exact_narrowing(gpu, oracle, tile, dt, use):
    """The stored tile equals RNE(in) bit for bit only if every element landed in the
    lane and slot the destination use assigns to it."""
    lh = gpu
    announce(f"coopmat_convert_use tile={tile} {dt} {use}")
    rng = np.random.default_rng(tile + len(use))
    ntiles = 5
    x = edge_values(rng, ntiles * tile * tile)
    inp = flat(lh, x, "f32")
    out = zeros(lh, x.size, dt)
    lh.coopmat_convert_use(inp.ptr, out.ptr, dt, tile, use, ntiles)
    got = out.to_numpy().view(np.uint16)
    ref = oracle.f32_to_f16_bits(x) if dt == "f16" else oracle.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(got, ref)


def test_convert_use_feeds_second_product(gpu, oracle):
    """D = convert(MatrixA f16, P) * V: the P_A step of a flash kernel, against the fp64
    product of the fp16-rounded P."""
    lh = gpu
    announce("coopmat_convert_use_muladd 16x16x16")
    rng = np.random.default_rng(9)
    ntiles = 8
    P = rng.uniform(0, 1, (ntiles, 16, 16)).astype(np.float32)
    V = rng.standard_normal((ntiles, 16, 16)).astype(np.float16)
    dP = flat(lh, np.concatenate([p.ravel(order="F") for p in P]), "f32")
    dV = flat(lh, np.concatenate([v.ravel(order="F") for v in V]), "f16")
    dD = zeros(lh, ntiles * 256, "f32")
    lh.coopmat_convert_use_muladd(dP.ptr, dV.ptr, dD.ptr, ntiles)
    got = dD.to_numpy().reshape(ntiles, 16, 16).transpose(0, 2, 1)
    for t in range(ntiles):
        ref = P[t].astype(np.float16).astype(np.float64) @ V[t].astype(np.float64)
        assert oracle.rel_frobenius(got[t], ref) <= 1e-6
        # the product of the unrounded P differs: the narrowing happened
        assert oracle.rel_frobenius(ref, P[t].astype(np.float64) @ V[t].astype(np.float64)) > 1e-6


@pytest.mark.parametrize("op", ["mul", "add"])
@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("layout", range(8))
def test_elementwise_layouts(gpu, oracle, op, tile, layout):
    """mul / add of two Accumulator tiles in every row/column-major combination, padded
    strides, several tiles: one fp32 operation per element, so bit-exact."""
    lh = gpu
    announce(f"coopmat_elementwise {op} tile={tile} layout={layout}")
    rng = np.random.default_rng(layout + 10 * tile)
    ntiles, sa, sb, sd = 3, tile + 5, tile + 2, tile + 9
    step = tile * max(sa, sb, sd) + 3
    n = step * ntiles + tile * max(sa, sb, sd)
    A = rng.standard_normal(n).astype(np.float32)
    B = rng.standard_normal(n).astype(np.float32)
    dA, dB, dD = flat(lh, A, "f32"), flat(lh, B, "f32"), zeros(lh, n, "f32")
    lh.coopmat_elementwise(op, tile, dA.ptr, sa, dB.ptr, sb, dD.ptr, sd, layout, ntiles, step)
    ref = np.zeros(n, np.float32)
    f = np.multiply if op == "mul" else np.add
    for t in range(ntiles):
        a = oracle.load_tile(A, t * step, sa, bool(layout & 1), tile, tile)
        b = oracle.load_tile(B, t * step, sb, bool(layout & 2), tile, tile)
        ref = oracle.store_tile(ref, t * step, sd, bool(layout & 4), f(a, b).astype(np.float32))
    np.testing.assert_array_equal(dD.to_numpy(), ref)


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("factor_rowmajor", [False, True])
def test_mul_stride_zero_factor_is_a_rescale(gpu, oracle, tile, factor_rowmajor):
    """coopmat_mul with a factor matrix loaded at stride 0: column-major gives the per-row
    rescale (attention's O *= alpha[row]), row-major the per-column one."""
    lh = gpu
    announce(f"coopmat_elementwise mul stride-0 factor tile={tile} rowmajor={factor_rowmajor}")
    rng = np.random.default_rng(21 + tile)
    m = rng.standard_normal((tile, tile)).astype(np.float32)
    v = rng.uniform(0.5, 2.0, tile).astype(np.float32)
    dM = flat(lh, m.ravel(order="F"), "f32")
    dV = flat(lh, v, "f32")
    dD = zeros(lh, tile * tile, "f32")
    layout = 2 if factor_rowmajor else 0
    lh.coopmat_elementwise("mul", tile, dM.ptr, tile, dV.ptr, 0, dD.ptr, tile, layout, 1, 0)
    got = dD.to_numpy().reshape(tile, tile).T
    ref = (m * (v[None, :] if factor_rowmajor else v[:, None])).astype(np.float32)
    np.testing.assert_array_equal(got, ref)


def test_accinit_muladd(gpu, oracle):
    """D = muladd(a, b, add(bias at stride 0, residual at ldr)): bias one value per row."""
    lh = gpu
    announce("coopmat_accinit_muladd 16x16x16")
    rng = np.random.default_rng(31)
    ntiles, ldr, ldd = 4, 21, 18
    A = rng.uniform(-1, 1, (ntiles, 16, 16)).astype(np.float16)
    B = rng.uniform(-1, 1, (ntiles, 16, 16)).astype(np.float16)
    bias = rng.standard_normal(16 * ntiles).astype(np.float32)
    Rm = rng.standard_normal((ldr, 16 * ntiles)).astype(np.float32)   # column-major, ld = ldr
    dA = flat(lh, np.concatenate([a.ravel(order="F") for a in A]), "f16")
    dB = flat(lh, np.concatenate([b.ravel(order="F") for b in B]), "f16")
    dbias = flat(lh, bias, "f32")
    dR = flat(lh, Rm.ravel(order="F"), "f32")
    dD = zeros(lh, ldd * 16 * ntiles, "f32")
    lh.coopmat_accinit_muladd(dA.ptr, dB.ptr, dbias.ptr, dR.ptr, ldr, dD.ptr, ldd, ntiles)
    D = dD.to_numpy().reshape(16 * ntiles, ldd).T
    for t in range(ntiles):
        c = A[t].astype(np.float64) @ B[t].astype(np.float64)
        ref = oracle.gemm_epilogue(c, bias=bias[16 * t:16 * t + 16], residual=Rm[:16, 16 * t:16 * t + 16])
        assert oracle.rel_frobenius(D[:16, 16 * t:16 * t + 16], ref) <= 1e-6
    assert np.all(D[16:] == 0)   # rows past the tile in the padded ld are not written


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("act", ["none", "relu", "gelu_tanh", "gelu_erf"])
def test_foreach_getcomp_setcomp(gpu, oracle, tile, act):
    """Every component visited once: gelu applied twice, or a component skipped, fails."""
    lh = gpu
    announce(f"coopmat_foreach_act tile={tile} act={act}")
    rng = np.random.default_rng(41 + tile)
    ntiles = 4
    x = (3 * rng.standard_normal(ntiles * tile * tile)).astype(np.float32)
    din, dout = flat(lh, x, "f32"), zeros(lh, x.size, "f32")
    dlen = zeros(lh, 1, "i32")
    lh.coopmat_foreach_act(din.ptr, dout.ptr, tile, act, ntiles, dlen.ptr)
    got = dout.to_numpy().astype(np.float64)
    ref = oracle.ACTS[act](x.astype(np.float64))
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) <= 2e-6
    assert int(dlen.to_numpy()[0]) == tile * tile // 64 == lh.coopmat_length("f32", tile, tile, "Accumulator")


def test_coopmat_length_table(gpu):
    lh = gpu
    announce("coopmat_length")
    for (dt, r, c, use) in [("f16", 16, 16, "MatrixA"), ("f16", 16, 32, "MatrixA"), ("f16", 32, 16, "MatrixA"),
                            ("f16", 16, 16, "MatrixB"), ("f16", 32, 16, "MatrixB"), ("f16", 16, 32, "MatrixB"),
                            ("i8", 16, 64, "MatrixA"), ("i8", 64, 16, "MatrixB"), ("f32", 16, 16, "Accumulator"),
                            ("f32", 32, 32, "Accumulator")]:
        assert lh.coopmat_length(dt, r, c, use) * 64 == r * c
    with pytest.raises(lh.Unsupported):
        lh.coopmat_length("f16", 8, 8, "MatrixA")


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("by_row", [False, True])
def test_perelement_pointer_extras(gpu, oracle, tile, by_row):
    """f(r, c, e, ptr, base): the fp16 per-column dequant scale of W8A16 and the fp32 per-row
    rescale of attention, both reading memory through the `extras` pointer at an offset."""
    lh = gpu
    announce(f"coopmat_perelement_scale tile={tile} by_row={by_row}")
    rng = np.random.default_rng(51 + tile + by_row)
    ntiles, base = 3, 5
    x = rng.standard_normal(ntiles * tile * tile).astype(np.float32)
    if by_row:
        fac = rng.standard_normal(base + ntiles * tile + 4).astype(np.float32)
        dfac = flat(lh, fac, "f32")
    else:
        fac = rng.uniform(0.001, 0.02, base + ntiles * tile + 4).astype(np.float16)
        dfac = flat(lh, fac, "f16")
    din, dout = flat(lh, x, "f32"), zeros(lh, x.size, "f32")
    lh.coopmat_perelement_scale(din.ptr, dout.ptr, tile, by_row, dfac.ptr, base, ntiles)
    got = dout.to_numpy().reshape(ntiles, tile, tile)
    for t in range(ntiles):
        m = x[t * tile * tile:(t + 1) * tile * tile].reshape(tile, tile, order="F")
        b = base + t * tile
        ref = oracle.scale_rows(m, fac, b) if by_row else oracle.scale_columns(m, fac, b)
        np.testing.assert_array_equal(got[t].T, ref)


# ---------------------------------------------------------------- caps()
def rocminfo_gpu_agent() -> dict:
    """The first gfx950 agent of `rocminfo` (the ROCm runtime's own report, read in a
    separate process): name, compute units, wavefront size, workgroup limit, LDS bytes."""
    import re
    import subprocess
    text = subprocess.run(["/opt/rocm/bin/rocminfo"], capture_output=True, text=True, timeout=60).stdout
    for block in text.split("*******"):
        if re.search(r"Name:\s+gfx950", block):
            def num(label):
                m = re.search(label + r":\s+(\d+)", block)
                return int(m.group(1)) if m else None
            lds = re.search(r"Segment:\s+GROUP\s+Size:\s+(\d+)\(0x[0-9a-f]+\) KB", block)
            return {"cus": num("Compute Unit"), "wave": num("Wavefront Size"),
                    "wg_max": num("Workgroup Max Size"), "lds": int(lds.group(1)) * 1024 if lds else None}
    raise AssertionError("rocminfo lists no gfx950 agent")


def test_caps_device_record(gpu):
    """caps() on the box: the fields come from hipDeviceProp of device 0 and agree with
    rocminfo's report of the same agent; the MFMA table answers the host queries."""
    lh = gpu
    announce("caps() device record")
    c = lh.caps()
    p = lh.vocabulary.device_properties()
    r = rocminfo_gpu_agent()
    assert c.coopmat and c.tile == 16 and c.subgroup == 64 and c.coopmatsubgroup == 64
    assert p["gfx_arch"] == 950
    assert c.cores == r["cus"] == 256
    assert c.subgroup == r["wave"]
    assert c.workgrouplimit == r["wg_max"] == 1024
    assert r["lds"] is None or c.sharedbudget == r["lds"]
    assert c.sharedbudget >= 64 * 1024
    assert c.warps >= 4 and c.warps * c.subgroup <= 64 * 64
    assert p["hbm_bytes"] > 250 * 2 ** 30 and p["l2_bytes"] >= 4 * 2 ** 20
    # the MFMA table answers the host queries the way Lava's callers ask them
    assert lh.bestshape(c, "f16", "f32") == lh.MatrixShape("f16", "f32", 16, 16, 16)
    assert lh.bestshape(c, "i8", "i32") == lh.MatrixShape("i8", "i32", 32, 32, 32)
    assert lh.bestshape(c, "f16", "f32", scope=lh.WorkgroupScope()) is None
    assert lh.supports(c, lh.MatrixShape("bf16", "f32", 32, 32, 16))
    assert lh.matrix_shapes(c.with_(coopmat=False)) == ()


def test_caps_wggran_rows_run(gpu, oracle):
    """Each wggran row is a workgroup-scope matrix the library runs: a GEMM at that many
    invocations with (M, N, K) at multiples of the row is exact to fp32 accumulation, and
    an extent that is not a multiple is refused."""
    lh = gpu
    c = lh.caps()
    assert c.wggran, "caps().wggran is empty"
    assert lh.wggranularity(c, 256) == (32, 32, 16)
    assert lh.wggranularity(c, 96) is None
    rng = np.random.default_rng(61)
    for (nt, gm, gn, gk) in c.wggran:
        M, N, K = 2 * gm, 3 * gn, 5 * gk
        for layout in (0, 7):
            announce(f"workgroup gemm nt={nt} M={M} N={N} K={K} layout={layout}")
            A = rng.uniform(-1, 1, (M, K)).astype(np.float16)
            B = rng.uniform(-1, 1, (K, N)).astype(np.float16)
            order = "C" if layout else "F"
            dA = lh.HIPDeviceArray.from_numpy(A, order=order)
            dB = lh.HIPDeviceArray.from_numpy(B, order=order)
            dC = lh.HIPDeviceArray("f32", (M, N), order=order)
            lh.coopmat_workgroup_gemm(dC, dA, dB, nt)
            ref = A.astype(np.float64) @ B.astype(np.float64)
            assert oracle.rel_frobenius(dC.to_numpy(), ref) <= 1e-6
        bad = lh.HIPDeviceArray("f16", (gm + 16 if gm > 16 else 8, K), order="F")
        dBad = lh.HIPDeviceArray("f32", (bad.dims[0], N), order="F")
        with pytest.raises(lh.InvalidArgument):
            lh.coopmat_workgroup_gemm(dBad, bad, lh.HIPDeviceArray("f16", (K, N), order="F"), nt)
