"""Shared pytest set-up: paths, the `gpu` marker, and device detection.

CPU tests (`-m "not gpu"`) cover the oracle against golden vectors and closed
forms, the host mirror of the vocabulary, and the C ABI's exports and argument
checks.  GPU tests (`-m gpu`) call liblava_hip.so through its C ABI and compare
with the oracle.  A missing library fails a GPU test; only a missing GPU skips it.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "lava.jl_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and liblava_hip.so")


_HAS_GPU = None


def has_gpu() -> bool:
    global _HAS_GPU
    if _HAS_GPU is None:
        import lava_hip
        try:
            _HAS_GPU = lava_hip.device_count() > 0
        except FileNotFoundError:
            raise
        except Exception:
            _HAS_GPU = False
    return _HAS_GPU


@pytest.fixture(scope="session")
def gpu():
    """The lava_hip module, initialised on a gfx950; skips only when no GPU exists."""
    import lava_hip
    lava_hip.load()   # a missing library is a failure, not a skip
    if not has_gpu():
        pytest.skip("no GPU visible")
    lava_hip.init()
    return lava_hip


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


def announce(msg: str) -> None:
    """Name the GPU case before running it, so a crash log says which one."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture
def rng():
    return np.random.default_rng(12345)


def _pinned_gemm(gpu, choice, name):
    gpu.set_kernel_override(gpu.FAMILY_GEMM, choice)
    gpu.kernel_log_clear()
    try:
        yield
        log = gpu.kernel_log()
    finally:
        gpu.set_kernel_override(gpu.FAMILY_GEMM, 0)
    assert name in log, f"expected {name} in the kernel log, got {log}"


@pytest.fixture
def tile_kernel(gpu):
    """Runs a test's GEMMs on the 256 x 256 tile kernel (pinned with lava_hip_set_kernel_override,
    so that the rate rule cannot move them to another kernel) and checks afterwards, through the
    library's kernel log, that it ran."""
    yield from _pinned_gemm(gpu, 1, "gemm_tn_kernel")


@pytest.fixture
def staged_kernel(gpu):
    """As tile_kernel, for the staged (any-layout, bounds-predicated) kernel."""
    yield from _pinned_gemm(gpu, 3, "gemm_staged_kernel")


@pytest.fixture
def mid_kernel(gpu):
    """As tile_kernel, for the 128 x 128 mid-size kernel."""
    yield from _pinned_gemm(gpu, 4, "gemm_mid_kernel")
