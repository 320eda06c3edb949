"""ctypes binding of liblava_hip.so (include/lava_hip.h).

The library is the product: every compute call below goes to a gfx950 kernel.
There is no CPU fallback; when the library or a GPU is missing the call raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liblava_hip.so"

OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_NO_DEVICE = -4

# element type codes
F16, BF16, F32, I8, U8, I32, U32, F64 = 0, 1, 2, 3, 4, 5, 6, 7
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2, 3

A_ROWMAJOR, B_ROWMAJOR, C_ROWMAJOR = 1, 2, 4

COMBINE_ADD, COMBINE_MAX, COMBINE_MIN = 0, 1, 2

USE_MATRIX_A, USE_MATRIX_B, USE_ACCUMULATOR = 0, 1, 2
ELEMENTWISE_MUL, ELEMENTWISE_ADD = 0, 1


class LavaHIPError(RuntimeError):
    """A nonzero status from liblava_hip.so, with its thread-local message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


class InvalidArgument(LavaHIPError, ValueError):
    pass


class Unsupported(LavaHIPError, NotImplementedError):
    pass


class NoDevice(LavaHIPError):
    pass


vp = C.c_void_p
i64 = C.c_int64
u32 = C.c_uint32
u64 = C.c_uint64
ci = C.c_int

# name -> (restype, argtypes)
PROTOTYPES: dict[str, tuple] = {
    "lava_hip_init": (ci, []),
    "lava_hip_device_count": (ci, [C.POINTER(ci)]),
    "lava_hip_malloc": (ci, [C.POINTER(vp), C.c_size_t]),
    "lava_hip_free": (ci, [vp]),
    "lava_hip_memcpy_h2d": (ci, [vp, vp, C.c_size_t]),
    "lava_hip_memcpy_d2h": (ci, [vp, vp, C.c_size_t]),
    "lava_hip_memcpy_d2d": (ci, [vp, vp, C.c_size_t, vp]),
    "lava_hip_fill_bytes": (ci, [vp, C.c_uint8, C.c_size_t, vp]),
    "lava_hip_synchronize": (ci, []),
    "lava_hip_stream_synchronize": (ci, [vp]),
    "lava_hip_stream_create": (ci, [C.POINTER(vp)]),
    "lava_hip_stream_destroy": (ci, [vp]),
    "lava_hip_event_create": (ci, [C.POINTER(vp)]),
    "lava_hip_event_destroy": (ci, [vp]),
    "lava_hip_event_record": (ci, [vp, vp]),
    "lava_hip_event_elapsed_ms": (ci, [C.POINTER(C.c_float), vp, vp]),
    "lava_hip_last_error": (C.c_char_p, []),
    "lava_hip_version": (ci, []),
    "lava_hip_device_caps": (ci, [C.POINTER(i64), ci]),
    "lava_hip_matrix_shapes": (ci, [C.POINTER(C.c_int32), ci, C.POINTER(ci)]),
    "lava_hip_fill_uniform": (ci, [vp, ci, i64, u64, C.c_double, C.c_double, vp]),
    "lava_hip_fill_normal": (ci, [vp, ci, i64, u64, vp]),
    "lava_hip_fill_i8": (ci, [vp, i64, u64, ci, vp]),
    "lava_hip_coopmat_muladd_16x16x16": (ci, [ci, ci, vp, i64, i64, vp, i64, i64, vp, i64, i64,
                                              vp, i64, i64, u32, i64, i64, vp]),
    "lava_hip_coopmat_perelement_rowcol": (ci, [vp, vp, ci, i64, vp]),
    "lava_hip_coopmat_perelement_pair": (ci, [vp, vp, vp, ci, i64, vp]),
    "lava_hip_coopmat_reduce": (ci, [vp, vp, ci, u32, ci, i64, vp]),
    "lava_hip_coopmat_reduce_into": (ci, [vp, vp, ci, ci, ci, u32, ci, i64, vp]),
    "lava_hip_coopmat_convert": (ci, [vp, vp, ci, i64, vp]),
    "lava_hip_dot4x8": (ci, [vp, vp, vp, i64, vp]),
    "lava_hip_coopmat_convert_use": (ci, [vp, vp, ci, ci, ci, i64, vp]),
    "lava_hip_coopmat_convert_use_muladd_16x16x16": (ci, [vp, vp, vp, i64, vp]),
    "lava_hip_coopmat_elementwise": (ci, [ci, ci, vp, i64, vp, i64, vp, i64, u32, i64, i64, vp]),
    "lava_hip_coopmat_accinit_muladd_16x16x16": (ci, [vp, vp, vp, vp, i64, vp, i64, i64, vp]),
    "lava_hip_coopmat_foreach_act": (ci, [vp, vp, ci, ci, i64, vp, vp]),
    "lava_hip_coopmat_length": (ci, [ci, ci, ci, ci, C.POINTER(C.c_int32)]),
    "lava_hip_coopmat_perelement_scale": (ci, [vp, vp, ci, ci, vp, i64, i64, vp]),
    "lava_hip_workgroup_shapes": (ci, [C.POINTER(C.c_int32), ci, C.POINTER(ci)]),
    "lava_hip_coopmat_workgroup_gemm_f16": (ci, [ci, vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_f16_f32": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_bf16_f32": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_i8_i32": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_u8_u32": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_coopmat_gemm_f16_tiles": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_ex": (ci, [ci, ci, vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp, vp, i64, ci, vp]),
    "lava_hip_tensor_load_tile": (ci, [ci, ci, vp, vp, ci, vp, vp, vp]),
    "lava_hip_tensor_store_tile": (ci, [ci, ci, vp, vp, vp, ci, vp]),
    "lava_hip_tensor_muladd_16x16x16": (ci, [vp, vp, vp, vp, ci, vp, vp]),
    "lava_hip_gemm_cm2_f16": (ci, [vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_w8a16": (ci, [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_gemm_w8a16_noalloc": (ci, [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, u32, vp]),
    "lava_hip_flash_attn_fwd_f16": (ci, [vp, vp, vp, vp, i64, i64, i64, i64, C.POINTER(i64),
                                         C.POINTER(i64), C.c_float, ci, vp]),
    "lava_hip_release_workspaces": (ci, []),
    "lava_hip_read_stream": (ci, [vp, C.c_size_t, vp, ci, ci, vp]),
    "lava_hip_mfma_loop": (ci, [ci, vp, vp, C.c_size_t, ci, ci, ci, vp, vp]),
    "lava_hip_graph_capture_begin": (ci, [vp]),
    "lava_hip_graph_capture_end": (ci, [vp, C.POINTER(vp)]),
    "lava_hip_graph_launch": (ci, [vp, vp]),
    "lava_hip_graph_destroy": (ci, [vp]),
    "lava_hip_kernel_log": (C.c_char_p, []),
    "lava_hip_kernel_log_clear": (None, []),
    "lava_hip_set_kernel_override": (ci, [ci, ci]),
}

# kernel families of lava_hip_set_kernel_override
FAMILY_ATTN, FAMILY_GEMM = 1, 2

_lib: C.CDLL | None = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load liblava_hip.so (once) and attach the prototypes.

    Raises FileNotFoundError if the library has not been built.
    """
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    lib = C.CDLL(str(p))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    msg = load().lava_hip_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    """Raise the matching LavaHIPError for a nonzero status."""
    if status == OK:
        return
    msg = last_error()
    cls = {ERR_INVALID_ARG: InvalidArgument, ERR_UNSUPPORTED: Unsupported,
           ERR_NO_DEVICE: NoDevice}.get(status, LavaHIPError)
    raise cls(status, msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def kernel_log() -> list[str]:
    """Names of the kernels this thread launched since the last kernel_log_clear()."""
    raw = load().lava_hip_kernel_log()
    return raw.decode().split("+") if raw else []


def kernel_log_clear() -> None:
    load().lava_hip_kernel_log_clear()


def set_kernel_override(family: int, choice: int) -> None:
    """Pin a family's kernel choice process-wide (0 = automatic); for tests and A/B timing."""
    call("lava_hip_set_kernel_override", family, choice)


def release_workspaces() -> None:
    """Free the library's workspaces (waits for the device first)."""
    call("lava_hip_release_workspaces")
