"""The BASELINE configs at their full sizes on the HIP device, against the CPU oracle.

C1 runs in tests/test_hip_runs.py, the full-length loss curves in tests/test_hip_curves.py.
Here C2, C3, C4 and C5 compile for "hip" at validation level 'standard', whose device check runs
one step on the oracle and on the device; every output of that step is also compared element
by element. Then the per-step losses of a few device-loop steps are overlaid on the oracle's
(1e-4 relative), and the resulting parameters compared. The oracle's 2-D products run row-parallel here (bit-identical to
its serial loop), so each config checks in well under a minute.
"""

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import workloads
from rustautograd_amd import tree as rtree

from helpers import close

pytestmark = pytest.mark.gpu


def _device_check(c, key_bias_d=None):
    """The compiled report's checks: finite, optimizer equivalence, and the device check. With
    attention present, a DEVICE_MISMATCH warning may only concern the key third of the
    projection bias (zero true gradient; see `_compare_outputs`); every output is then compared
    element by element by `_compare_outputs`, since the device check reports one mismatch only
    (validate.rs:698)."""
    checks = {k["name"]: k for k in c.report["checks"]}
    assert checks["finite"]["status"] == "pass", checks["finite"]
    assert checks["optimizer_equivalence"]["status"] == "pass", checks["optimizer_equivalence"]
    dev = checks["device_equivalence"]
    if key_bias_d is None:
        assert dev["status"] == "pass", dev
        assert c.report.ok, c.report["diagnostics"]
        return dev
    names = c._out_def.paths("out")
    for d in c.report["diagnostics"]:
        assert d["code"] == "DEVICE_MISMATCH", d
        name, element = names[d["observation"]["output_index"]], d["observation"]["element"]
        assert name.endswith("attn.qkv.b") and key_bias_d <= element < 2 * key_bias_d, d
    return dev


def _without_key_bias(name, values, key_bias_d):
    """A parameter's values with the attention key bias third removed (kept for every other
    leaf). That third's true gradient is exactly zero, since softmax ignores a per-row shift of
    the scores: both sides compute rounding noise there, which AdamW scales to +-lr."""
    if key_bias_d is not None and name.endswith("attn.qkv.b"):
        return np.concatenate([values[:key_bias_d], values[2 * key_bias_d:]])
    return values


def _compare_outputs(gpu, cpu, state, key_bias_d, tol=1e-4):
    """Every output of one step on the device against the oracle's, element by element."""
    a, b = gpu(state), cpu(state)
    for (name, u), (_, v) in zip(rtree.paths(a, "out."), rtree.paths(b, "out.")):
        close(_without_key_bias(name, u.numpy(), key_bias_d), _without_key_bias(name, v.numpy(), key_bias_d), tol, name)


def _overlay(step, state, steps, key_bias_d=None):
    print(f"compile for hip and cpu, {steps} steps", flush=True)
    gpu = rg.compile(step, (state,), validate="standard", device="hip")
    cpu = rg.compile(step, (state,), validate="none", device="cpu")
    _device_check(gpu, key_bias_d)
    _compare_outputs(gpu, cpu, state, key_bias_d)
    a = rg.run(gpu, state, steps=steps)
    b = rg.run(cpu, state, steps=steps)
    assert a.status == b.status == "completed"
    close(np.array(a.history["aux"]), np.array(b.history["aux"]), 1e-4, "loss curve")
    for (name, u), (_, v) in zip(rtree.paths(a.state["params"]), rtree.paths(b.state["params"])):
        close(_without_key_bias(name, u.numpy(), key_bias_d), _without_key_bias(name, v.numpy(), key_bias_d), 1e-4, name)
    return a, b


def test_c2_mlp_full_size():
    """C2: 4096 x 512 -> 2048 -> 2048 -> 1, gelu, AdamW; x drawn in-graph each step."""
    step, state = workloads.mlp_train_step(workloads.MLPConfig())
    _overlay(step, state, 3)


@pytest.mark.parametrize("name,steps", [("C3", 3), ("C4", 2)])
def test_gpt_full_size(name, steps):
    """C3 (tied embeddings) and C4 (the headline) at full size: device check, every output of
    one step element by element, the loss overlay and the parameters after the loop, all with
    only the key third of the projection bias left out."""
    cfg = workloads.GPT_CONFIGS[name]
    step, state = workloads.gpt_train_step(cfg)
    _overlay(step, state, steps, key_bias_d=cfg.d)


def test_c5_matrix_chain_full_size():
    """C5: sum(((A@B)@C)@D) and its gradients for B and C; n = 4096, k = 8."""
    program, inputs = workloads.matrix_chain()
    gpu = rg.compile(program, inputs, validate="standard", device="hip")
    _device_check(gpu)
    cpu = rg.compile(program, inputs, validate="none", device="cpu")
    (value, gb, gc), (cv, cb, cc) = gpu(*inputs), cpu(*inputs)
    # The gradients are small (~1e-3): compare relative to their own largest magnitude.
    for name, u, v in (("dB", gb, cb), ("dC", gc, cc)):
        u, v = u.numpy().astype(np.float64), v.numpy().astype(np.float64)
        err = np.abs(u - v).max() / np.abs(v).max()
        assert err <= 1e-4, f"{name}: {err:.2e} relative to max|cpu|"
    # The value sums 64 cancelling products of 4096-term chains.
    assert abs(float(value) - float(cv)) <= 1e-3 * abs(float(cv)), (float(value), float(cv))
