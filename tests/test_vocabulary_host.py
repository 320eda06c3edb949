"""Host half of the vocabulary (src/vocabulary/matrix.jl, caps.jl) on CPU:
shape ordering, table queries, and the DeviceCaps copy rules.
"""
from __future__ import annotations

import pytest

import lava_hip as lh
from lava_hip import DeviceCaps, MatrixShape, SubgroupScope, WorkgroupScope


def S(ab, acc, m, n, k, scope=None):
    return MatrixShape(ab, acc, m, n, k, scope or SubgroupScope())


def test_bestshape_is_squarest_then_largest():
    table = [S("f16", "f32", 16, 16, 32), S("f16", "f32", 32, 32, 16), S("f16", "f32", 16, 16, 16),
             S("f16", "f32", 32, 32, 8), S("i8", "i32", 16, 16, 16)]
    assert lh.bestshape(table, "f16", "f32") == S("f16", "f32", 16, 16, 16)
    # among equally square shapes the larger wins
    tie = [S("f16", "f32", 16, 16, 32), S("f16", "f32", 32, 32, 16)]
    assert lh.bestshape(tie, "f16", "f32") == S("f16", "f32", 32, 32, 16)
    # the type pair must match exactly, and scope too
    assert lh.bestshape(table, "bf16", "f32") is None
    assert lh.bestshape(table, "f16", "f32", WorkgroupScope()) is None


def test_shape_identity_and_supports():
    a, b = S("f16", "f32", 16, 16, 16), S("f16", "f32", 16, 16, 16)
    assert a == b and hash(a) == hash(b)
    assert a != S("f16", "f16", 16, 16, 16)
    assert a != S("f16", "f32", 16, 16, 16, WorkgroupScope())
    assert lh.supports([a], b) and not lh.supports([a], S("i8", "i32", 16, 16, 16))


def test_devicecaps_defaults_and_copy_rules():
    c = DeviceCaps(True, 16, 64, 64, 65536, 1024, 256, 8)
    assert c.shapes == (S("f16", "f32", 16, 16, 16),)
    assert lh.matrix_shapes(c) == c.shapes
    off = c.with_(coopmat=False)
    # the copy changes exactly the named field: the table is kept, the accessor gates it
    assert off.shapes == c.shapes and lh.matrix_shapes(off) == ()
    assert not lh.supports(off, S("f16", "f32", 16, 16, 16))
    assert lh.bestshape(off, "f16", "f32") is None
    none = DeviceCaps(False, 16, 64, 64, 65536, 1024, 256, 8)
    assert none.shapes == ()


def test_wggranularity_table_lookup():
    c = DeviceCaps(True, 16, 32, 32, 49152, 1024, 48, 48, wggran=[(128, 32, 16, 16), (256, 32, 32, 16)])
    assert lh.wggranularity(c, 256) == (32, 32, 16)
    assert lh.wggranularity(c, 64) is None


def test_gfx950_table_answers():
    table = lh.library_shapes()
    assert lh.bestshape(table, "f16", "f32") == S("f16", "f32", 16, 16, 16)
    assert lh.bestshape(table, "bf16", "f32") == S("bf16", "f32", 16, 16, 16)
    assert lh.bestshape(table, "i8", "i32") == S("i8", "i32", 32, 32, 32)
    assert lh.bestshape(table, "u8", "u32") is None   # CDNA4 has no unsigned MFMA
    assert lh.bestshape(table, "f64", "f64") == S("f64", "f64", 16, 16, 4)
    assert lh.bestshape(table, "f32", "f32") == S("f32", "f32", 16, 16, 4)
    assert lh.supports_coopmat_perelement() and lh.supports_coopmat_reduce()
    assert lh.CoopMatReduce.Row == 1 and lh.CoopMatReduce.RowAndColumn == 3


def test_workgroup_layout_of_vectors():
    """test_workgroup_vector_layout.jl:24-27: <2 x half> 4/4, <4 x half> 8/8, <2 x float> 8/8,
    <4 x float> 16/16 -- and the rule's other cases (3 components packed, aligned as 4)."""
    assert lh.workgroup_layout("f16", 2) == (4, 4)
    assert lh.workgroup_layout("f16", 4) == (8, 8)
    assert lh.workgroup_layout("f32", 2) == (8, 8)
    assert lh.workgroup_layout("f32", 4) == (16, 16)
    assert lh.workgroup_layout("f32", 3) == (12, 16)
    assert lh.workgroup_layout("f16", 1) == (2, 2)
    assert lh.workgroup_layout("i8", 4) == (4, 4)
    with pytest.raises(ValueError):
        lh.workgroup_layout("f32", 5)
