"""Device arrays and streams over liblava_hip.so's hipMalloc/hipMemcpy wrappers.

`HIPDeviceArray` is the host-side counterpart of Lava's kernel argument
`LavaDeviceArray{T,N}(ptr, dims)` (src/device/devicearray.jl:35-38): a device
address plus its dimensions, column-major by default as in Julia
(src/device/devicearray.jl:138-174).  `order="C"` gives a row-major array for
callers that lay their data out that way.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import _lib

try:  # numpy has no bfloat16: carry its bits as uint16
    _BF16 = np.dtype("uint16")
except Exception:  # pragma: no cover
    _BF16 = None

# logical element type -> (code, numpy storage dtype)
DTYPES = {
    "f16": (_lib.F16, np.dtype(np.float16)),
    "bf16": (_lib.BF16, np.dtype(np.uint16)),
    "f32": (_lib.F32, np.dtype(np.float32)),
    "i8": (_lib.I8, np.dtype(np.int8)),
    "u8": (_lib.U8, np.dtype(np.uint8)),
    "i32": (_lib.I32, np.dtype(np.int32)),
    "u32": (_lib.U32, np.dtype(np.uint32)),
    "f64": (_lib.F64, np.dtype(np.float64)),
}


def _prod(dims: Sequence[int]) -> int:
    n = 1
    for d in dims:
        n *= int(d)
    return n


class HIPDeviceArray:
    """A device allocation of `prod(dims)` elements of `dtype`, freed on close/GC."""

    def __init__(self, dtype: str, dims: Sequence[int], order: str = "F"):
        if dtype not in DTYPES:
            raise ValueError(f"unknown element type {dtype!r}; one of {sorted(DTYPES)}")
        if order not in ("F", "C"):
            raise ValueError("order must be 'F' (column-major) or 'C' (row-major)")
        self.dtype = dtype
        self.code, self.np_dtype = DTYPES[dtype]
        self.dims = tuple(int(d) for d in dims)
        if any(d < 0 for d in self.dims):
            raise ValueError(f"negative dimension in {self.dims}")
        self.order = order
        self.nbytes = _prod(self.dims) * self.np_dtype.itemsize
        p = C.c_void_p()
        _lib.call("lava_hip_malloc", C.byref(p), self.nbytes)
        self._ptr = p.value or 0

    # -- identity ---------------------------------------------------------
    @property
    def ptr(self) -> int:
        return self._ptr

    @property
    def size(self) -> int:
        return _prod(self.dims)

    def pointer(self, i: int = 1) -> int:
        """Address of element `i` (1-based, linear), as `pointer(a, i)` in Julia."""
        return self._ptr + (i - 1) * self.np_dtype.itemsize

    def strides(self) -> tuple[int, ...]:
        """Element strides of each dimension."""
        st, acc = [], 1
        dims = self.dims if self.order == "F" else tuple(reversed(self.dims))
        for d in dims:
            st.append(acc)
            acc *= d
        return tuple(st) if self.order == "F" else tuple(reversed(st))

    # -- transfers --------------------------------------------------------
    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype: str | None = None, order: str = "F") -> "HIPDeviceArray":
        if dtype is None:
            dtype = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.int8): "i8",
                     np.dtype(np.uint8): "u8", np.dtype(np.int32): "i32", np.dtype(np.uint32): "u32",
                     np.dtype(np.float64): "f64"}.get(a.dtype)
            if dtype is None:
                raise ValueError(f"pass dtype= for numpy dtype {a.dtype}")
        out = cls(dtype, a.shape, order)
        out.copy_from(a)
        return out

    def copy_from(self, a: np.ndarray) -> None:
        if a.shape != self.dims:
            raise ValueError(f"shape {a.shape} != {self.dims}")
        host = np.asarray(a).astype(self.np_dtype, copy=False)
        host = np.asfortranarray(host) if self.order == "F" else np.ascontiguousarray(host)
        if self.nbytes:
            _lib.call("lava_hip_memcpy_h2d", self._ptr, host.ctypes.data, self.nbytes)

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self.dims, dtype=self.np_dtype, order=self.order)
        if self.nbytes:
            _lib.call("lava_hip_memcpy_d2h", out.ctypes.data, self._ptr, self.nbytes)
        return out

    def fill_bytes(self, value: int = 0, stream: int | None = None) -> None:
        _lib.call("lava_hip_fill_bytes", self._ptr, value, self.nbytes, stream)

    # -- lifetime ---------------------------------------------------------
    def close(self) -> None:
        if self._ptr:
            _lib.call("lava_hip_free", self._ptr)
            self._ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __repr__(self) -> str:
        return f"HIPDeviceArray({self.dtype}, {self.dims}, order={self.order!r}, ptr=0x{self._ptr:x})"


class Stream:
    """A non-blocking HIP stream (default priority)."""

    def __init__(self):
        s = C.c_void_p()
        _lib.call("lava_hip_stream_create", C.byref(s))
        self.handle = s.value

    def synchronize(self) -> None:
        _lib.call("lava_hip_stream_synchronize", self.handle)

    def close(self) -> None:
        if self.handle:
            _lib.call("lava_hip_stream_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        _lib.call("lava_hip_event_create", C.byref(e))
        self.handle = e.value

    def record(self, stream: int | None = None) -> None:
        _lib.call("lava_hip_event_record", self.handle, stream)

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        _lib.call("lava_hip_event_elapsed_ms", C.byref(ms), self.handle, later.handle)
        return float(ms.value)

    def close(self) -> None:
        if self.handle:
            _lib.call("lava_hip_event_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """A HIP graph captured from the library's calls on a (non-NULL) stream:

        g = Graph(stream)
        with g.capture():
            gemm(C, A, B, stream=stream.handle)
        g.launch()

    Capture is in global mode, so an allocating call anywhere in the process fails while it runs."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.handle = None

    def capture(self):
        graph = self

        class _Capture:
            def __enter__(self_):
                _lib.call("lava_hip_graph_capture_begin", graph.stream.handle)
                return graph

            def __exit__(self_, exc_type, exc, tb):
                e = C.c_void_p()
                status = _lib.load().lava_hip_graph_capture_end(graph.stream.handle, C.byref(e))
                graph.handle = e.value
                if exc_type is None:
                    _lib.check(status)
                return False

        return _Capture()

    def launch(self, stream: Stream | None = None) -> None:
        _lib.call("lava_hip_graph_launch", self.handle, (stream or self.stream).handle)

    def close(self) -> None:
        if self.handle:
            _lib.call("lava_hip_graph_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synchronize() -> None:
    _lib.call("lava_hip_synchronize")


def device_count() -> int:
    n = C.c_int()
    _lib.call("lava_hip_device_count", C.byref(n))
    return n.value
