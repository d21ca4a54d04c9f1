"""Loads the engine module and the HIP device backend built in this package.

The engine (`_rg`, C++) drives device libraries through the C ABI of include/rg_hip.h. The
product registers exactly one: librg_hip.so, as device "hip". When it is missing or no gfx950
device is present, compiling for "hip" fails with a DEVICE_UNAVAILABLE diagnostic that says
why; nothing falls back to the CPU.
"""

import ctypes
import json
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIBRARY = os.path.join(_HERE, "lib", "librg_hip.so")

try:
    from . import _rg
except ImportError as e:  # pragma: no cover - reported with the build command
    raise ImportError(f"rustautograd_amd engine module is not built ({e}); run __graft_entry__.build()") from e

DiagnosticError = _rg.DiagnosticError

_hip_error = None
_hip_lib = None


def _register_hip():
    global _hip_error, _hip_lib
    if not os.path.exists(HIP_LIBRARY):
        _hip_error = f"{HIP_LIBRARY} is not built; run __graft_entry__.build()"
        return
    try:
        _rg.register_backend("hip", HIP_LIBRARY, "rg_hip_")
        _hip_lib = ctypes.CDLL(HIP_LIBRARY)
        if not _hip_lib.rg_hip_available():
            _hip_error = "librg_hip.so loaded, but no gfx950 device is visible to HIP"
    except ImportError as e:
        _hip_error = str(e)


_register_hip()


def hip_error():
    """Why the HIP backend is unusable in this process, or None."""
    return _hip_error


def require(device):
    """Raises a DEVICE_UNAVAILABLE diagnostic naming why `device` cannot be used."""
    detail = _hip_error if device == "hip" else f"no backend named {device!r} is registered"
    d = {
        "status": "validation_failed", "severity": "error", "code": "DEVICE_UNAVAILABLE",
        "node": None, "observation": {"device": device, "available": list(_rg.available_devices()), "detail": detail},
        "diagnosis": {"cause": "unknown_device" if device != "hip" else "hip_backend_unavailable", "certainty": "verified"},
    }
    err = DiagnosticError(json.dumps(d))
    err.diagnostic = d
    raise err


def register_backend(name, path, prefix):
    """Registers another library with the same C ABI under `name` (used by test harnesses)."""
    _rg.register_backend(name, os.path.abspath(path), prefix)


def device_memory_bytes(device):
    """Memory of the device a plan runs on, for the near-capacity warning; None if unknown."""
    if device == "hip" and _hip_lib is not None and not _hip_error:
        f = _hip_lib.rg_hip_device_memory_bytes
        f.restype = ctypes.c_uint64
        return int(f())
    return None
