"""Build liblava_hip.so from lava.jl_amd/csrc/*.hip for gfx950 (in-tree).

`python -m lava_hip.build` (with lava.jl_amd on sys.path) or
`__graft_entry__.build()`.  Every HIP source is compiled with hipcc for gfx950
only; packed fp32 instructions are disabled (`-packed-fp32-ops`).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent            # lava.jl_amd/
REPO = ROOT.parent               # repository root
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "liblava_hip.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> tuple[Path, str]:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMPILE_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "is not a recognized feature for this target" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    return obj, err


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link liblava_hip.so. Always recompiles."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; liblava_hip.so needs the ROCm toolchain")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    objs = [o for o, _ in results]
    if verbose:
        for (o, msg) in results:
            if msg.strip():
                print(f"[{o.name}] {msg}", file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
