"""Host half of Lava's cooperative-matrix vocabulary, answered for MI355X.

Mirrors src/vocabulary/matrix.jl and src/vocabulary/caps.jl: the operand
positions (`MatrixA`, `MatrixB`, `Accumulator`), scopes, the `MatrixShape` table a
device reports, `supports`/`bestshape` over it, and `DeviceCaps` with its copy
constructor.  `caps()` asks liblava_hip.so for the gfx950 answer.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field, replace
from typing import Iterable, Optional, Sequence


# ---- MatrixUse / MatrixScope (src/vocabulary/matrix.jl:37-66) ----------------
class MatrixUse:
    name = "MatrixUse"

    def __repr__(self) -> str:
        return self.name


class _MatrixA(MatrixUse):
    name = "MatrixA"


class _MatrixB(MatrixUse):
    name = "MatrixB"


class _Accumulator(MatrixUse):
    name = "Accumulator"


MatrixA, MatrixB, Accumulator = _MatrixA(), _MatrixB(), _Accumulator()


class MatrixScope:
    name = "MatrixScope"

    def __repr__(self) -> str:
        return self.name

    def __eq__(self, other) -> bool:
        return type(self) is type(other)

    def __hash__(self) -> int:
        return hash(type(self).__name__)


class SubgroupScope(MatrixScope):
    name = "SubgroupScope"


class WorkgroupScope(MatrixScope):
    name = "WorkgroupScope"


# ---- CoopMatReduce (src/vocabulary/coopmat.jl:292-297) -----------------------
class CoopMatReduce:
    Row = 1
    Column = 2
    RowAndColumn = 3
    TwoByTwo = 4


# dtype names <-> liblava_hip.so codes
_CODE_NAMES = {0: "f16", 1: "bf16", 2: "f32", 3: "i8", 4: "u8", 5: "i32", 6: "u32", 7: "f64"}


# ---- MatrixShape (src/vocabulary/matrix.jl:88-113) -----------------------------
@dataclass(frozen=True)
class MatrixShape:
    """One (M, N, K) the hardware implements for operands `ab` accumulating in `acc`."""
    ab: str
    acc: str
    M: int
    N: int
    K: int
    scope: MatrixScope = field(default_factory=SubgroupScope)

    def __eq__(self, other) -> bool:
        return (isinstance(other, MatrixShape) and self.ab == other.ab and self.acc == other.acc
                and self.M == other.M and self.N == other.N and self.K == other.K
                and type(self.scope) is type(other.scope))

    def __hash__(self) -> int:
        return hash((self.ab, self.acc, self.M, self.N, self.K, type(self.scope).__name__))

    def __repr__(self) -> str:
        return f"MatrixShape({self.ab}->{self.acc} {self.M}x{self.N}x{self.K} {self.scope!r})"


def supports(shapes_or_caps, s: MatrixShape) -> bool:
    """Whether `s` is in the table (src/vocabulary/matrix.jl:135)."""
    shapes = matrix_shapes(shapes_or_caps) if isinstance(shapes_or_caps, DeviceCaps) else shapes_or_caps
    return any(x == s for x in shapes)


def isbetter(a: MatrixShape, b: MatrixShape) -> bool:
    """Squarest, then largest (src/vocabulary/matrix.jl:166-173)."""
    sa = abs(a.M - a.N) + abs(a.N - a.K)
    sb = abs(b.M - b.N) + abs(b.N - b.K)
    if sa != sb:
        return sa < sb
    return a.M * a.N * a.K > b.M * b.N * b.K


def bestshape(shapes_or_caps, ab: str, acc: str, scope: MatrixScope | None = None) -> Optional[MatrixShape]:
    """The shape to use for ab -> acc at `scope`, or None (src/vocabulary/matrix.jl:155-164)."""
    scope = scope if scope is not None else SubgroupScope()
    shapes = matrix_shapes(shapes_or_caps) if isinstance(shapes_or_caps, DeviceCaps) else shapes_or_caps
    best = None
    for s in shapes:
        if not (s.ab == ab and s.acc == acc and type(s.scope) is type(scope)):
            continue
        if best is None or isbetter(s, best):
            best = s
    return best


# ---- DeviceCaps (src/vocabulary/caps.jl:54-108) ----------------------------------
@dataclass(frozen=True)
class DeviceCaps:
    coopmat: bool
    tile: int
    subgroup: int
    coopmatsubgroup: int
    sharedbudget: int
    workgrouplimit: int
    cores: int
    warps: int
    wggran: tuple = ()
    shapes: Optional[tuple] = None

    def __post_init__(self):
        # The 8/9-argument form means "a device with a square `tile` fp16 -> fp32
        # instruction" (caps.jl:73-82): give it that one-entry table.
        if self.shapes is None:
            object.__setattr__(self, "shapes", (MatrixShape("f16", "f32", self.tile, self.tile, self.tile),)
                               if self.coopmat else ())
        else:
            object.__setattr__(self, "shapes", tuple(self.shapes))
        object.__setattr__(self, "wggran", tuple(tuple(x) for x in self.wggran))

    def with_(self, **kw) -> "DeviceCaps":
        """`DeviceCaps(c; kw...)`: the same caps with the named fields replaced and
        nothing else moved (caps.jl:84-108)."""
        return replace(self, **kw)


def matrix_shapes(c) -> tuple:
    """The coopmat gate lives here, not in the copy constructor (caps.jl:150-159)."""
    if isinstance(c, DeviceCaps):
        return c.shapes if c.coopmat else ()
    return tuple(c)


def wggranularity(c: DeviceCaps, nt: int):
    """(M, N, K) multiples of a workgroup-scope matrix at nt invocations, or None (caps.jl:140-145)."""
    for (n, m, nn, k) in c.wggran:
        if n == nt:
            return (m, nn, k)
    return None


def supports_coopmat_perelement(backend=None) -> bool:
    """Implemented natively on MI355X (lava_coopmat.hpp `perelement`)."""
    return True


def supports_coopmat_reduce(backend=None) -> bool:
    """Implemented natively on MI355X for Row, Column and RowAndColumn masks."""
    return True


def supports_flexible_coopmat_shapes(backend=None) -> bool:
    """Subgroup fragments are the MFMA shapes in the table.  The one place another extent is
    taken is the destination of a reduce (lava_hip_coopmat_reduce_into: 16, 32 or 64 along a
    free axis, half the extents for TwoByTwo), which is not the general capability this names."""
    return False


def supports_tensor_addressing(backend=None) -> bool:
    """The tensor-addressing vocabulary (layouts, clamp modes, slices, the transposing
    view; tensor.jl:109-115) is implemented natively: lava_tensor.hpp on the device,
    lava_hip.tensor on the host."""
    return True


_SCALAR_BYTES = {"f16": 2, "bf16": 2, "f32": 4, "f64": 8, "i8": 1, "u8": 1, "i16": 2, "i32": 4, "u32": 4, "i64": 8}


def workgroup_layout(elem: str, n: int = 1) -> tuple:
    """(size, alignment) in bytes of an n-component vector of `elem` in workgroup memory
    (LDS), the rule Lava's emitter applies to `@localmem` (src/compiler/spirv/types.jl:
    838-900, test/test_workgroup_vector_layout.jl:24-27): the components packed, aligned
    to 2x the component for 2 components and 4x for 3 or 4 (Vulkan's rule); a scalar is
    its own size.  The 2- and 4-component device types the kernels stage in LDS follow
    it (static_asserts in lava_coopmat.hpp)."""
    if elem not in _SCALAR_BYTES:
        raise ValueError(f"unknown component type {elem!r}")
    if n not in (1, 2, 3, 4):
        raise ValueError("vectors have 2, 3 or 4 components")
    b = _SCALAR_BYTES[elem]
    if n == 1:
        return b, b
    return n * b, (2 if n == 2 else 4) * b


_CAPS_FIELDS = ("coopmat", "tile", "subgroup", "coopmatsubgroup", "sharedbudget", "workgrouplimit", "cores",
                "warps", "clock_khz", "hbm_bytes", "l2_bytes", "gfx_arch")


def device_properties() -> dict:
    """Raw capability record of device 0 from liblava_hip.so (needs a GPU)."""
    from . import _lib
    out = (C.c_int64 * len(_CAPS_FIELDS))()
    _lib.call("lava_hip_device_caps", out, len(_CAPS_FIELDS))
    return dict(zip(_CAPS_FIELDS, (int(v) for v in out)))


def library_shapes() -> tuple:
    """The gfx950 MFMA shape table compiled into liblava_hip.so (no GPU needed)."""
    from . import _lib
    n = C.c_int()
    _lib.call("lava_hip_matrix_shapes", None, 0, C.byref(n))
    buf = (C.c_int32 * (6 * n.value))()
    _lib.call("lava_hip_matrix_shapes", buf, n.value, C.byref(n))
    rows = []
    for i in range(n.value):
        ab, acc, M, N, K, sc = buf[6 * i:6 * i + 6]
        rows.append(MatrixShape(_CODE_NAMES[ab], _CODE_NAMES[acc], M, N, K,
                                SubgroupScope() if sc == 0 else WorkgroupScope()))
    return tuple(rows)


def library_wggran() -> tuple:
    """The workgroup-scope table compiled into liblava_hip.so, rows (invocations, M, N, K):
    a workgroup of `invocations` lanes holds the matrix as invocations/64 wavefronts of
    16 x 16 MFMA tiles (no GPU needed)."""
    from . import _lib
    n = C.c_int()
    _lib.call("lava_hip_workgroup_shapes", None, 0, C.byref(n))
    buf = (C.c_int32 * (4 * n.value))()
    _lib.call("lava_hip_workgroup_shapes", buf, n.value, C.byref(n))
    return tuple(tuple(int(x) for x in buf[4 * i:4 * i + 4]) for i in range(n.value))


def caps() -> DeviceCaps:
    """`caps(backend)` for the MI355X this process sees (needs a GPU): the device record
    from hipDeviceProp, the MFMA shape table and the workgroup-scope table."""
    p = device_properties()
    return DeviceCaps(coopmat=bool(p["coopmat"]), tile=p["tile"], subgroup=p["subgroup"],
                      coopmatsubgroup=p["coopmatsubgroup"], sharedbudget=p["sharedbudget"],
                      workgrouplimit=p["workgrouplimit"], cores=p["cores"], warps=p["warps"],
                      wggran=library_wggran(), shapes=library_shapes())
