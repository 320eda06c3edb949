"""The C ABI on the CPU: liblava_hip.so loads, exports every entry point
include/lava_hip.h declares, and rejects bad arguments with a status and a
readable message before touching a device (no compute call needs a GPU here).
"""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "lava_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lava_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_functions()
    for required in ("lava_hip_gemm_f16_f32", "lava_hip_gemm_bf16_f32", "lava_hip_gemm_i8_i32",
                     "lava_hip_gemm_w8a16", "lava_hip_flash_attn_fwd_f16", "lava_hip_coopmat_muladd_16x16x16",
                     "lava_hip_coopmat_perelement_rowcol", "lava_hip_coopmat_reduce", "lava_hip_malloc",
                     "lava_hip_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import lava_hip
    lib = lava_hip.load()
    out = subprocess.run(["nm", "-D", "--defined-only", str(lava_hip._lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (lava_hip_\w+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # and the ctypes prototypes cover exactly the declared set
    assert sorted(lava_hip._lib.PROTOTYPES) == declared_functions()
    for n in declared_functions():
        getattr(lib, n)


def test_library_is_gfx950_only():
    """The offload bundle of our own build names gfx950 and no other target."""
    import lava_hip
    blob = lava_hip._lib.LIB_PATH.read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-[a-z]*-(gfx[0-9a-f]+)", blob))
    assert targets == {b"gfx950"}


def status_of(fn, *args):
    import lava_hip
    return getattr(lava_hip.load(), fn)(*args), lava_hip._lib.last_error()


def test_version_and_shapes_without_gpu():
    import lava_hip
    assert lava_hip.load().lava_hip_version() >= 100
    shapes = lava_hip.library_shapes()
    assert any(s.ab == "bf16" and s.M == 16 and s.K == 32 for s in shapes)
    assert any(s.ab == "i8" and s.acc == "i32" and s.K == 64 for s in shapes)


def test_gemm_argument_errors():
    i64 = C.c_int64
    rc, msg = status_of("lava_hip_gemm_bf16_f32", None, None, None, -1, 4, 4, 4, 4, 4, 7, None)
    assert rc == -1 and "negative extent" in msg
    rc, msg = status_of("lava_hip_gemm_bf16_f32", 16, 16, 16, 4, 4, 4, 4, 4, 4, 8, None)
    assert rc == -1 and "layout" in msg
    rc, msg = status_of("lava_hip_gemm_f16_f32", 16, 16, None, 4, 4, 4, 4, 4, 4, 7, None)
    assert rc == -1 and "null C" in msg
    rc, msg = status_of("lava_hip_gemm_i8_i32", 16, 16, 16, 8, 8, 8, 4, 8, 8, 7, None)
    assert rc == -1 and "lda" in msg
    rc, msg = status_of("lava_hip_gemm_i8_i32", 16, 16, 16, 8, 8, 8, 8, 8, 4, 7, None)
    assert rc == -1 and "ldc" in msg
    rc, msg = status_of("lava_hip_gemm_f16_f32", 17, 16, 16, 8, 8, 8, 8, 8, 8, 7, None)
    assert rc == -1 and "aligned" in msg
    # empty problems are no-ops that succeed without a device
    rc, _ = status_of("lava_hip_gemm_f16_f32", None, None, None, 0, 5, 5, 5, 5, 5, 7, None)
    assert rc == 0
    rc, msg = status_of("lava_hip_coopmat_gemm_f16_tiles", 16, 16, 16, 20, 16, 16, 16, 16, 16, 7, None)
    assert rc == -1 and "multiples" in msg


def test_w8a16_and_attention_argument_errors():
    rc, msg = status_of("lava_hip_gemm_w8a16", 16, 16, 16, 16, 16, 128, 256, 256, 100, 128, 7, None)
    assert rc == -1 and "ldw" in msg
    rc, msg = status_of("lava_hip_gemm_w8a16", 16, 16, None, 16, 16, 128, 256, 256, 128, 128, 7, None)
    assert rc == -1 and "null" in msg
    st = (C.c_int64 * 4)(2, 256, 256 * 128, 256 * 128 * 2)
    rc, msg = status_of("lava_hip_flash_attn_fwd_f16", 16, 16, 16, 16, 1, 2, 128, 128, st, None, C.c_float(0.1), 1,
                        None)
    assert rc == -1 and "contiguous" in msg
    st = (C.c_int64 * 4)(1, 128, 128 * 128, 128 * 128 * 2)
    rc, msg = status_of("lava_hip_flash_attn_fwd_f16", 16, 16, 16, 16, 1, 2, 128, 512, st, None, C.c_float(0.1), 1,
                        None)
    assert rc == -1 and "sequence stride" in msg
    st = (C.c_int64 * 4)(1, 512, 512 * 128, 512 * 128 * 2)
    rc, msg = status_of("lava_hip_flash_attn_fwd_f16", 16, 16, 16, 16, 1, 2, 128, 512, st, None,
                        C.c_float(float("nan")), 1, None)
    assert rc == -1 and "finite" in msg
    rc, msg = status_of("lava_hip_flash_attn_fwd_f16", 16, 16, 16, 16, 1, 2, 128, 300, st, None, C.c_float(0.1), 1,
                        None)
    assert rc == -2 and "D = 300" in msg
    rc, _ = status_of("lava_hip_flash_attn_fwd_f16", None, None, None, None, 0, 2, 128, 128, None, None,
                      C.c_float(0.1), 1, None)
    assert rc == 0


def test_vocabulary_argument_errors():
    rc, msg = status_of("lava_hip_coopmat_reduce", 16, 16, 16, 4, 1, 1, None)
    assert rc == -2 and "TwoByTwo" in msg
    rc, msg = status_of("lava_hip_coopmat_reduce", 16, 16, 24, 1, 1, 1, None)
    assert rc == -1 and "tile" in msg
    rc, msg = status_of("lava_hip_coopmat_muladd_16x16x16", 1, 2, 16, 1, 16, 16, 1, 16, 16, 1, 16, 16, 1, 16, 0, 1,
                        0, None)
    assert rc == -2 and "type pair" in msg
    rc, msg = status_of("lava_hip_coopmat_muladd_16x16x16", 0, 2, 16, 0, 16, 16, 1, 16, 16, 1, 16, 16, 1, 16, 0, 1,
                        0, None)
    assert rc == -1 and "1-based" in msg
    rc, msg = status_of("lava_hip_coopmat_convert", 16, 16, 0, 100, None)
    assert rc == -1 and "multiple of 256" in msg
    rc, msg = status_of("lava_hip_fill_uniform", 16, 7, 10, 1, C.c_double(0), C.c_double(1), None)
    assert rc == -1 and "dtype" in msg


def test_python_errors_are_typed():
    import lava_hip
    with pytest.raises(lava_hip.InvalidArgument):
        lava_hip.gemm_raw("bf16", "f32", 16, 16, 16, -1, 1, 1, 1, 1, 1, 7)
    with pytest.raises(lava_hip.Unsupported):
        lava_hip.gemm_raw("f32", "f32", 16, 16, 16, 1, 1, 1, 1, 1, 1, 7)


def test_vocabulary_queries_without_gpu():
    """coopmat_length and the workgroup-scope table are host queries of the library."""
    import lava_hip as lh
    assert lh.coopmat_length("f32", 16, 16, "Accumulator") == 4
    assert lh.coopmat_length("f32", 32, 32, "Accumulator") == 16
    assert lh.coopmat_length("f16", 16, 32, "MatrixA") == 8
    assert lh.coopmat_length("i8", 16, 64, "MatrixA") == 16
    with pytest.raises(lh.Unsupported):
        lh.coopmat_length("f16", 48, 16, "MatrixA")
    rows = lh.library_wggran()
    assert rows[0] == (64, 16, 16, 16)
    for nt, m, n, k in rows:
        # nt / 64 wavefronts of 16 x 16 tiles, K in steps of the 16x16x16 instruction
        assert (m // 16) * (n // 16) * 64 == nt and k == 16
    # coarsening: a larger workgroup never asks for smaller multiples
    for a, b in zip(rows, rows[1:]):
        assert b[0] > a[0] and b[1] >= a[1] and b[2] >= a[2]
    c = lh.DeviceCaps(True, 16, 64, 64, 163840, 1024, 256, 32, wggran=rows)
    assert lh.wggranularity(c, 512) == (64, 32, 16) and lh.wggranularity(c, 100) is None


def test_vocabulary_entry_argument_errors():
    import lava_hip as lh
    L = lh.load()
    st, msg = status_of("lava_hip_coopmat_convert_use", None, None, lh._lib.F16, 8, 0, 1, None)
    assert st == lh._lib.ERR_INVALID_ARG and "tile" in msg
    st, msg = status_of("lava_hip_coopmat_convert_use", None, None, lh._lib.F32, 16, 0, 1, None)
    assert st == lh._lib.ERR_INVALID_ARG and "dtype" in msg
    st, msg = status_of("lava_hip_coopmat_elementwise", 7, 16, None, 0, None, 0, None, 16, 0, 1, 0, None)
    assert st == lh._lib.ERR_INVALID_ARG and "op" in msg
    st, msg = status_of("lava_hip_coopmat_elementwise", 0, 16, 8, -1, 8, 0, 8, 16, 0, 1, 0, None)
    assert st == lh._lib.ERR_INVALID_ARG and "stride" in msg
    st, msg = status_of("lava_hip_coopmat_foreach_act", None, None, 16, 9, 1, None, None)
    assert st == lh._lib.ERR_INVALID_ARG and "act" in msg
    st, msg = status_of("lava_hip_coopmat_workgroup_gemm_f16", 96, None, None, None, 16, 16, 16, 16, 16, 16, 0, None)
    assert st == lh._lib.ERR_UNSUPPORTED and "96" in msg
    st, msg = status_of("lava_hip_coopmat_workgroup_gemm_f16", 256, 8, 8, 8, 48, 32, 16, 48, 16, 48, 0, None)
    assert st == lh._lib.ERR_INVALID_ARG and "multiples" in msg
    # zero tiles is a no-op that needs no device
    assert L.lava_hip_coopmat_perelement_scale(None, None, 16, 0, None, 0, 0, None) == 0
