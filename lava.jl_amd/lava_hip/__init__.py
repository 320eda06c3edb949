"""lava_hip -- MI355X (gfx950) implementation of Lava.jl's cooperative-matrix path.

The compute lives in liblava_hip.so (hand-written HIP kernels, C ABI in
include/lava_hip.h).  This package is its Python host mirror: loader, device
arrays, the host half of the vocabulary, and destination-first kernel calls.
"""
from . import _lib
from ._lib import (FAMILY_ATTN, FAMILY_GEMM, InvalidArgument, LavaHIPError, NoDevice, Unsupported, kernel_log,
                   kernel_log_clear, load, release_workspaces, set_kernel_override)
from .device import Event, Graph, HIPDeviceArray, Stream, device_count, synchronize
from .kernels import (coopmat_accinit_muladd, coopmat_convert, coopmat_convert_use, coopmat_convert_use_muladd,
                      coopmat_elementwise, coopmat_foreach_act, coopmat_gemm_tiles, coopmat_length,
                      coopmat_muladd_16x16x16, coopmat_perelement_pair, coopmat_perelement_rowcol,
                      coopmat_perelement_scale, coopmat_reduce, coopmat_reduce_into, coopmat_workgroup_gemm, dot4x8, fill_i8, fill_normal,
                      fill_uniform, flash_attn_fwd, flash_attn_fwd_raw, gemm, gemm_ex, gemm_ex_raw, gemm_raw, w8a16,
                      w8a16_noalloc, w8a16_raw)
from .tensor import (TENSOR_CLAMP_CONSTANT, TENSOR_CLAMP_TO_EDGE, TENSOR_CLAMP_UNDEFINED, TensorLayout, TensorView,
                     gemm_cm2, tensor_clampbits, tensor_layout, tensor_load_tile, tensor_muladd_16x16x16,
                     tensor_setclampvalue, tensor_setdim, tensor_setstride, tensor_slice, tensor_store_tile,
                     tensor_view)
from .vocabulary import (Accumulator, CoopMatReduce, DeviceCaps, MatrixA, MatrixB, MatrixShape, SubgroupScope,
                         WorkgroupScope, bestshape, caps, isbetter, library_shapes, library_wggran, matrix_shapes, supports,
                         supports_coopmat_perelement, supports_coopmat_reduce, supports_flexible_coopmat_shapes,
                         supports_tensor_addressing, wggranularity, workgroup_layout)

# Input seeds: base "LAVA" + 256 * config index + tensor id (A=0, B=1, scale=2; Q=0, K=1, V=2).
SEED_BASE = 0x4C415641


def seed(config: int, tensor: int) -> int:
    return SEED_BASE + 256 * config + tensor


def init() -> None:
    """Check that device 0 is a gfx950 (raises NoDevice otherwise)."""
    _lib.call("lava_hip_init")
