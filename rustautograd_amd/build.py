"""Builds the native parts of rustautograd_amd in-tree.

    python -m rustautograd_amd.build          # engine module + librg_hip.so (gfx950)

- `_rg*.so`: the C++ engine (graph, autodiff, optimizer, planner, validation, run loop) as a
  pybind11 module, built with g++.
- `lib/librg_hip.so`: the HIP device backend (include/rg_hip.h), built with hipcc for gfx950.
  Every HIP translation unit is compiled with packed fp32 instructions disabled and without
  floating-point contraction; fused groups are compiled at run time with the same options.

Compilation cross-compiles without a GPU, so this runs anywhere ROCm is installed.
"""

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
BUILD = os.path.join(ROOT, "_build")

ENGINE_SOURCES = ["graph.cpp", "autodiff.cpp", "optimize.cpp", "egraph.cpp", "plan.cpp", "attention.cpp", "backend.cpp", "validate.cpp",
                  "module.cpp"]
HIP_SOURCES = ["kernels.hip", "gemm.hip", "attention.hip", "noalloc.hip", "runtime.cpp", "jit.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result",
             # MFMA accumulators in ordinary VGPRs: without it the GEMM's pipelined loop copies every
             # accumulator out of and back into AGPRs on each iteration.
             "-mllvm", "-amdgpu-mfma-vgpr-form"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def _pybind_includes():
    import pybind11
    return ["-I" + pybind11.get_include(), "-I" + sysconfig.get_paths()["include"]]


def build_engine():
    os.makedirs(os.path.join(BUILD, "engine"), exist_ok=True)
    src = os.path.join(CSRC, "engine")
    inc = _pybind_includes()
    objs = []

    def compile_one(name):
        obj = os.path.join(BUILD, "engine", name + ".o")
        _run(["g++", "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-sign-compare", *inc, "-c",
              os.path.join(src, name), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, ENGINE_SOURCES))
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(HERE, "_rg" + suffix)
    _run(["g++", "-shared", "-o", out, *objs, "-ldl"])
    return out


def build_hip():
    os.makedirs(os.path.join(BUILD, "hip"), exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    src = os.path.join(CSRC, "hip")

    def compile_one(name):
        obj = os.path.join(BUILD, "hip", name + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(src, name), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    out = os.path.join(LIB, "librg_hip.so")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out, *objs, "-L/opt/rocm/lib", "-lhiprtc",
          "-Wl,-rpath,/opt/rocm/lib"])
    return out


def build_all():
    with ThreadPoolExecutor(max_workers=2) as ex:
        f1 = ex.submit(build_engine)
        f2 = ex.submit(build_hip)
        return f1.result(), f2.result()


if __name__ == "__main__":
    for p in build_all():
        print("built", p)
    sys.exit(0)
