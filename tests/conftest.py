"""Test harness: registers the CPU oracle as device "cpu" (the parity checker) and the `gpu` marker.

The oracle (oracle/cpu_exec.cpp) implements the device C ABI on the CPU. Tests compile the same
program for "hip" (the product) and "cpu" (the oracle) and compare results; CPU-only tests also
use it to exercise the engine, since the product has no CPU executor.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

ORACLE = os.path.join(ROOT, "oracle", "_build", "librg_cpu.so")
# The oracle registered a second time under another name: the engine plans for a device (split
# sums, level order, absorbed broadcasts, device fusion) for every backend not named "cpu", so
# this runs the HIP-flavoured plan on the CPU oracle.
DEVPLAN = "cpu_devplan"


def _ensure_built():
    """Builds the engine module and the oracle when a fresh checkout lacks them."""
    import glob
    import subprocess
    if not glob.glob(os.path.join(ROOT, "rustautograd_amd", "_rg*.so")):
        sys.path.insert(0, ROOT)
        from rustautograd_amd import build
        build.build_engine()
    if not os.path.exists(ORACLE):
        subprocess.run(["bash", os.path.join(ROOT, "oracle", "build.sh")], check=True)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the HIP backend")
    _ensure_built()
    from rustautograd_amd import _native
    _native.register_backend("cpu", ORACLE, "rg_cpu_")
    _native.register_backend(DEVPLAN, ORACLE, "rg_cpu_")
    # The checker splits large 2-D products over rows (bit-identical to the reference's serial
    # loop, tests/test_engine.py checks it), so full-size configs can be checked in seconds.
    import ctypes
    ctypes.CDLL(ORACLE).rg_cpu_set_row_parallel_gemm(1)


@pytest.fixture(autouse=True)
def _default_device(request):
    """Tests without the gpu marker run the engine on the CPU oracle; gpu tests use "hip"."""
    from rustautograd_amd import program
    saved = program.DEFAULT_DEVICE
    program.DEFAULT_DEVICE = "hip" if "gpu" in request.keywords else "cpu"
    yield
    program.DEFAULT_DEVICE = saved


def pytest_collection_modifyitems(config, items):
    import rustautograd_amd as rg
    if "hip" in rg.devices():
        return
    skip = pytest.mark.skip(reason="no gfx950 device with the HIP backend in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def oracle_threads():
    """Sets the CPU oracle's thread count for a test, restoring it afterwards."""
    import ctypes
    lib = ctypes.CDLL(ORACLE)
    saved = lib.rg_cpu_threads()
    yield lambda n: lib.rg_cpu_set_threads(int(n))
    lib.rg_cpu_set_threads(saved)
