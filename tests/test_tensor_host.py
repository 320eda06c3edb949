"""The host half of the tensor-addressing vocabulary (lava_hip/tensor.py), no GPU.

Mirrors src/vocabulary/tensor.jl: tensor_layout / tensor_setdim (packed strides, the
whole tensor as the slice) / tensor_setstride / tensor_setclampvalue / tensor_slice /
tensor_clampbits (tensor.jl:83-85: the bits of x in T, zero-extended) / tensor_view,
and the plain struct the C ABI takes.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import lava_hip as lh


def test_setdim_packs_and_slices_whole():
    l = lh.tensor_setdim(lh.tensor_layout(3, lh.TENSOR_CLAMP_CONSTANT), (4, 5, 6))
    assert l.dims == (4, 5, 6)
    assert l.strides == (30, 6, 1)          # innermost last, packed
    assert l.offsets == (0, 0, 0) and l.sizes == (4, 5, 6)
    assert l.clamp == lh.TENSOR_CLAMP_CONSTANT and l.clampbits == 0


def test_layouts_are_values():
    """Each builder returns a new layout (Lava's are SSA values), the input is unchanged."""
    a = lh.tensor_setdim(lh.tensor_layout(2), (8, 8))
    b = lh.tensor_slice(a, (1, 2), (3, 4))
    c = lh.tensor_setstride(b, (16, 1))
    d = lh.tensor_setclampvalue(c, 7)
    assert a.offsets == (0, 0) and a.sizes == (8, 8) and a.strides == (8, 1)
    assert b.offsets == (1, 2) and b.sizes == (3, 4) and b.strides == (8, 1)
    assert c.strides == (16, 1) and c.offsets == (1, 2)
    assert d.clampbits == 7 and c.clampbits == 0


def test_clampbits_match_tensor_jl():
    # Float16: Int32(reinterpret(UInt16, Float16(x))) -- 1.0 is 0x3C00, -2.0 is 0xC000 (zero-extended)
    assert lh.tensor_clampbits(1.0, "f16") == 0x3C00
    assert lh.tensor_clampbits(-2.0, "f16") == 0xC000
    # Float32: the IEEE bits as a signed Int32
    assert lh.tensor_clampbits(1.0, "f32") == 0x3F800000
    assert lh.tensor_clampbits(-1.0, "f32") == np.array([-1.0], np.float32).view(np.int32)[0]
    # integers: Int32(x)
    assert lh.tensor_clampbits(-3, "i8") == -3 and lh.tensor_clampbits(9, "i32") == 9
    with pytest.raises(ValueError):
        lh.tensor_clampbits(1.0, "bf16")


def test_struct_matches_the_c_header():
    l = lh.tensor_slice(lh.tensor_setclampvalue(lh.tensor_setdim(lh.tensor_layout(2, 2), (10, 20)), -1),
                        (-3, 4), (16, 8))
    c = l.to_c()
    assert ctypes.sizeof(c) == 3 * 4 + 4 * 16      # rank, clamp, clampbits, 4 x int32[4]
    assert (c.rank, c.clamp, c.clampbits) == (2, 2, 0xFFFFFFFF)
    assert list(c.dim)[:2] == [10, 20] and list(c.stride)[:2] == [20, 1]
    assert list(c.off)[:2] == [-3, 4] and list(c.size)[:2] == [16, 8]


def test_views_and_argument_errors():
    assert lh.tensor.__name__.endswith("tensor")
    assert lh.tensor._transpose_flag(None, 2) == 0
    assert lh.tensor._transpose_flag(lh.tensor_view(2, (0, 1)), 2) == 0
    assert lh.tensor._transpose_flag(lh.tensor_view(2, (1, 0)), 2) == 1
    assert lh.tensor._transpose_flag(lh.tensor_view(3, (0, 2, 1)), 3) == 1
    with pytest.raises(lh.Unsupported):
        lh.tensor._transpose_flag(lh.tensor_view(3, (2, 1, 0)), 3)
    with pytest.raises(ValueError):
        lh.tensor_view(2, (0, 0))
    with pytest.raises(ValueError):
        lh.tensor._transpose_flag(lh.tensor_view(2, (1, 0)), 3)
    with pytest.raises(ValueError):
        lh.tensor_layout(5)
    with pytest.raises(ValueError):
        lh.tensor_layout(2, 3)
    with pytest.raises(ValueError):
        lh.tensor_setdim(lh.tensor_layout(2), (1, 2, 3))
    with pytest.raises(ValueError):
        lh.tensor_setdim(lh.tensor_layout(2), (-1, 2))
    with pytest.raises(ValueError):
        lh.tensor_slice(lh.tensor_setdim(lh.tensor_layout(2), (4, 4)), (0, 0), (2, -1))
    with pytest.raises(ValueError):
        lh.tensor_setdim(lh.tensor_layout(2), (2 ** 31, 1))


def test_supports_tensor_addressing():
    assert lh.supports_tensor_addressing() is True
