"""The drop-in boundary: the C ABI of include/rg_hip.h, checked without a GPU.

librg_hip.so must load on a host without a device, export every entry point the header declares,
report itself unavailable rather than crash, and compile a plan's fused kernels for gfx950
through hiprtc (which needs no device). The CPU oracle implements the same ABI under the
`rg_cpu_` prefix, which is what lets the engine drive either library.
"""

import ctypes
import json
import os
import re

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import _native, _rg, workloads
from helpers import G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rg_hip.h")
PLAN_HEADER = os.path.join(ROOT, "include", "rg_plan.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(rg_hip_[a-z_]+)\s*\(", text)))


def test_header_declares_the_full_surface():
    names = _declared()
    for required in ("rg_hip_available", "rg_hip_program_new", "rg_hip_program_free", "rg_hip_exec_new", "rg_hip_exec_free",
                     "rg_hip_exec_write", "rg_hip_exec_read", "rg_hip_exec_scalar", "rg_hip_exec_swap", "rg_hip_exec_step",
                     "rg_hip_exec_failure", "rg_hip_exec_step_timed", "rg_hip_exec_breakdown", "rg_hip_exec_run",
                     "rg_hip_program_allocated_bytes", "rg_hip_program_inject_failure"):
        assert required in names


def test_hip_library_loads_and_exports_every_declared_symbol():
    assert os.path.exists(_native.HIP_LIBRARY), "librg_hip.so is not built"
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"librg_hip.so lacks {missing}"


# Entry points the engine binds as optional (backend.cpp), with a host-side fallback each: the
# per-step timer, the JSON breakdown, the class timer and the device-resident run loop (the oracle uses the
# engine's host run loop, validate.rs:289-363), plus the HIP-only build check and memory query, and
# the run loop for callers that cannot allocate (a device-only entry point the engine does not bind).
OPTIONAL = {"rg_hip_exec_step_timed", "rg_hip_exec_breakdown", "rg_hip_exec_run", "rg_hip_exec_time_steps", "rg_hip_compile_check",
            "rg_hip_device_memory_bytes", "rg_hip_exec_run_noalloc", "rg_hip_gemm_streamed", "rg_hip_device_peaks",
            "rg_hip_kernel_source", "rg_hip_program_step_runs_in"}


def test_oracle_implements_the_same_abi():
    from conftest import ORACLE
    lib = ctypes.CDLL(ORACLE)
    missing = [n for n in _declared() if n not in OPTIONAL and not hasattr(lib, n.replace("rg_hip_", "rg_cpu_"))]
    assert not missing, f"oracle lacks {missing}"


def test_plan_header_enums_are_dense():
    """Op codes are a dense enum ending in RG_OP_COUNT, which the descriptor parser relies on."""
    text = open(PLAN_HEADER).read()
    body = re.search(r"enum rg_op\s*\{(.*?)\}", text, re.S).group(1)
    names = [re.match(r"\s*(RG_OP_[A-Z0-9_]+)", part).group(1) for part in body.split(",") if part.strip()]
    values = [int(v) for v in re.findall(r"=\s*(\d+)", body)]
    assert names[0] == "RG_OP_INPUT" and values[0] == 0
    assert names[-1] == "RG_OP_COUNT" and len(set(names)) == len(names)


@pytest.mark.skipif(rg.devices().count("hip") > 0, reason="a device is present: the gpu tests cover it")
def test_without_a_device_the_product_fails_loudly():
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    assert lib.rg_hip_available() == 0
    assert _native.hip_error()
    with pytest.raises(rg.DiagnosticError) as e:
        rg.compile(lambda x: x * 2.0, (rg.tensor(np.ones(3, np.float32)),), device="hip")
    d = e.value.diagnostic
    assert d["code"] == "DEVICE_UNAVAILABLE" and d["observation"]["device"] == "hip"
    assert "hip" not in rg.devices()


def test_product_package_never_touches_the_oracle():
    """Only tests/, smoke() and the bench's CPU baseline may use oracle/."""
    pkg = os.path.join(ROOT, "rustautograd_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".h", ".hip")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text and "rg_cpu_" not in text, f"{f} references the oracle"


def _compile_check(words):
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    f = lib.rg_hip_compile_check
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t]
    arr = (ctypes.c_int64 * len(words))(*words)
    err = ctypes.create_string_buffer(8192)
    n = f(arr, len(words), err, len(err))
    return n, err.value.decode()


def test_fused_kernels_of_a_small_program_compile_for_gfx950():
    """The generated HIP source of every fused group builds with hiprtc for gfx950."""
    g = G()
    x = g.input((64, 300), "float32")
    b = g.input((300,), "float32")
    h = g.un("tanh", g.bin("add", x, b))
    y = g.sum_all(g.bin("mul", g.un("exp", h), h))
    gx = g.grad(y, [x])[0]
    words, _ = _rg.plan_words(g.g, [y, gx], "hip", "standard")
    n, err = _compile_check(words)
    assert n >= 1, err


def test_kernels_inside_control_flow_bodies_compile_for_gfx950():
    """A scan's body is planned like a program: its fused groups are generated and compiled
    too (the nested plan descriptors of include/rg_plan.h)."""
    b = G()
    c, x = b.input((64, 300), "float32"), b.input((64, 300), "float32")
    nxt = b.un("tanh", b.bin("add", b.bin("mul", c, x), x))
    g = G()
    c0, xs = g.input((64, 300), "float32"), g.input((5, 64, 300), "float32")
    node = g.g.scan(b.g, [nxt, b.un("exp", nxt)], 1, 1, 5, [c0, xs])
    last = g.g.output(node, 0, [64, 300], "float32")
    words_body, _ = _rg.plan_words(g.g, [last], "hip", "standard")
    n_body, err = _compile_check(words_body)
    assert n_body >= 1, err


def _step_words(step, state):
    from rustautograd_amd import _pytree
    from rustautograd_amd.tensor import Tracer, lift, tracing
    leaves, in_def = _pytree.flatten((state,))
    g = _rg.Graph()
    tracers = [Tracer(g, g.input(list(t.shape), t.dtype, None)) for t in leaves]
    with tracing(g):
        out = step(*_pytree.unflatten(in_def, tracers))
        ids = [lift(g, leaf, "float32") for leaf in _pytree.leaves(out)]
    words, _ = _rg.plan_words(g, ids, "hip", "search-linear")
    return words


def _kernel_source(words):
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    buf = ctypes.create_string_buffer(8 << 20)
    arr = (ctypes.c_int64 * len(words))(*words)
    n = lib.rg_hip_kernel_source(arr, len(words), buf, len(buf))
    assert n >= 0, buf.value[:500]
    return buf.value.decode()


def test_product_epilogue_kernels_compile_for_gfx950(monkeypatch):
    """An elementwise group that reads a product of at least 1024 tiles (8192 x 1024 outputs) is
    generated as that product's epilogue (the tile of gemm_mfma.h compiled with hiprtc), and the
    program's kernels compile; with RG_HIP_EPILOGUE=0 every group keeps its own kernel. In C2 only
    the first layer's product has 1024 tiles (its activation, two adjacent columns per lane on an
    N-contiguous weight); RG_HIP_EPILOGUE=all takes the 512-tile ones too: the second layer's
    activation, the activation gradient (four adjacent columns per lane) and an AdamW update in
    a weight gradient's epilogue."""
    g = G()
    x, w = g.input((8192, 256), "float32"), g.input((256, 1024), "float32")
    y = g.op("matmul", [x, w])
    z = g.un("tanh", g.bin("mul", y, y))
    words, _ = _rg.plan_words(g.g, [z], "hip", "standard")
    src = _kernel_source(words)
    assert src.count("rgg::gemm_mfma_block<") == 1 and "amdgpu_waves_per_eu(2)" in src and "colp" not in src
    n, err = _compile_check(words)
    assert n >= 1, err
    # A column sum of the group's output (a bias gradient's shape) is computed by the same kernel
    # when the product's right operand is K-contiguous (its lanes hold runs of four columns).
    g = G()
    x, w = g.input((8192, 256), "float32"), g.input((1024, 256), "float32")
    y = g.op("matmul", [x, g.op("transpose", [w], perm=[1, 0])])
    z = g.un("tanh", g.bin("mul", y, y))
    zs = g.op("sum", [z], axes=[0], keepdims=False)
    words, _ = _rg.plan_words(g.g, [z, zs], "hip", "standard")
    src = _kernel_source(words)
    assert src.count("rgg::gemm_mfma_block<") == 1 and "colp[" in src
    n, err = _compile_check(words)
    assert n >= 1, err
    monkeypatch.setenv("RG_HIP_EPILOGUE", "0")
    assert "rgg::gemm_mfma_block<" not in _kernel_source(words)
    step, state = workloads.mlp_train_step()
    monkeypatch.delenv("RG_HIP_EPILOGUE")
    words = _step_words(step, state)
    assert _kernel_source(words).count("rgg::gemm_mfma_block<") == 1
    monkeypatch.setenv("RG_HIP_EPILOGUE", "all")
    src = _kernel_source(words)
    assert src.count("rgg::gemm_mfma_block<") == 4, src.count("rgg::gemm_mfma_block<")
    n, err = _compile_check(words)
    assert n >= 5, err


def test_c3_program_compiles_for_gfx950():
    """Every fused kernel of a whole GPT training step (C3 at reduced depth) compiles."""
    cfg = workloads.GPT_CONFIGS["C3"]._replace(batch=2, block=16, layers=1)
    step, state = workloads.gpt_train_step(cfg)
    from rustautograd_amd import _pytree
    from rustautograd_amd.tensor import Tracer, lift, tracing
    leaves, in_def = _pytree.flatten((state,))
    g = _rg.Graph()
    tracers = [Tracer(g, g.input(list(t.shape), t.dtype, None)) for t in leaves]
    with tracing(g):
        out = step(*_pytree.unflatten(in_def, tracers))
        ids = [lift(g, leaf, "float32") for leaf in _pytree.leaves(out)]
    words, _ = _rg.plan_words(g, ids, "hip", "search-linear")
    n, err = _compile_check(words)
    assert n >= 10, err


def test_standard_validation_without_a_cpu_reference_says_the_device_check_was_skipped():
    """With no CPU interpreter registered (the product alone ships none), validate='standard'
    cannot compare the device with the CPU: the report marks the check skipped and carries a
    DEVICE_CHECK_SKIPPED warning rather than passing silently. Run in a child process whose only
    backend is the oracle registered under another name, standing in for a device."""
    import subprocess
    import sys
    from conftest import ORACLE
    code = f"""
import json, sys
sys.path.insert(0, {ROOT!r})
import numpy as np
import rustautograd_amd as rg
from rustautograd_amd import _native
_native.register_backend("stand_in", {ORACLE!r}, "rg_cpu_")
c = rg.compile(lambda x: (x * 2.0).sum(), (rg.tensor(np.ones(4, np.float32)),), validate="standard", device="stand_in")
check = next(k for k in c.report["checks"] if k["name"] == "device_equivalence")
print(json.dumps([check["status"], [d["code"] for d in c.report["diagnostics"]], c.report["status"]]))
"""
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    status, codes, overall = json.loads(out.stdout.strip().splitlines()[-1])
    assert status == "skipped" and codes == ["DEVICE_CHECK_SKIPPED"] and overall == "warning"


def test_plans_reaching_past_their_slots_are_refused_by_both_backends():
    """The shared parser checks every slot reference and extent (rg_plan.h `check_refs`): a plan
    whose slots are too small for its steps, or whose output names a slot it does not have, is
    refused by the HIP library and by the oracle before any buffer is touched."""
    g = G()
    x = g.input((64, 300), "float32")
    y = g.sum_all(g.un("exp", g.un("tanh", x)))
    words, blob = _rg.plan_words(g.g, [y, g.grad(y, [x])[0]], "hip", "standard")
    assert _compile_check(list(words))[0] >= 1
    n_slots = words[2]
    shrunk = list(words)
    for s in range(n_slots):
        shrunk[3 + 3 * s + 1] = 1  # every slot's capacity down to one value
    misnamed = list(words)
    k = 3 + 3 * n_slots
    k += 1 + 3 * misnamed[k]  # constants
    k += 1 + 2 * misnamed[k]  # inputs
    misnamed[k + 1] = n_slots + 5  # the first output's slot
    oracle = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "librg_cpu.so"))
    oracle.rg_cpu_program_new.restype = ctypes.c_void_p
    oracle.rg_cpu_program_new.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t,
                                          ctypes.c_char_p, ctypes.c_size_t]
    for bad in (shrunk, misnamed):
        n, err = _compile_check(bad)
        assert n == -1 and "plan descriptor:" in err, (n, err)
        arr = (ctypes.c_int64 * len(bad))(*bad)
        msg = ctypes.create_string_buffer(4096)
        assert not oracle.rg_cpu_program_new(arr, len(bad), blob, len(blob), msg, len(msg))
        assert b"plan descriptor:" in msg.value, msg.value
