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


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the HIP backend")
    from rustautograd_amd import _native
    _native.register_backend("cpu", ORACLE, "rg_cpu_")


def pytest_collection_modifyitems(config, items):
    import rustautograd_amd as rg
    if "hip" in rg.devices():
        return
    skip = pytest.mark.skip(reason="no gfx950 device with the HIP backend in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
