"""The BASELINE configs at their full sizes on the HIP device, against the CPU oracle.

C1 runs in tests/test_hip_runs.py, the full-length loss curves in tests/test_hip_curves.py.
Here C2, C3, C4 and C5 compile for "hip" at validation level 'standard', whose device check runs
one step on the oracle and on the device. Then, each against the oracle:

- the gradients of the first step (the configs' `loss_and_grads` programs, the same draws as
  the step): every leaf within GRAD_TOL of that leaf's own largest magnitude;
- one whole training step: the loss at LOSS_TOL relative; AdamW's moments per leaf within
  GRAD_TOL of the leaf's largest moment; every parameter's update (new - old) by
  `helpers.updates_agree`, which takes out what the two sides' own moments explain;
- a few device-loop steps: the per-step losses at LOSS_TOL, and each parameter's movement over
  the run (new - initial), per leaf, within MOVE_TOL relative in the L2 norm. After more than
  one step the moments that explain an element's update are not at hand, and an element whose
  gradient sits near zero can move by up to the learning rate either way on rounding noise;
  the norm over the leaf bounds the aggregate, which a systematic error (a wrong update rule,
  a missing term) moves by its own size.

The attention key bias third (`attn.qkv.b[d:2d]`) is left out of every comparison: its true
gradient is exactly zero, since softmax ignores a per-row shift of the scores, so both sides
hold rounding noise there (~1e-9), which AdamW scales to the learning rate. Its q and v thirds
are compared. The oracle's 2-D products run row-parallel here (bit-identical to its serial
loop), so each config checks in well under a minute.

`DEVICE` is the device under test; the same checks run on the CPU against the device-flavoured
plan (`cpu_devplan`) in tests/test_config_checks.py, at reduced sizes.
"""

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import workloads
from rustautograd_amd import tree as rtree

from helpers import close_rel, updates_agree

pytestmark = pytest.mark.gpu

DEVICE = "hip"
GRAD_TOL = 1e-4
LOSS_TOL = 1e-5
MOVE_TOL = 1e-3


def _device_check(c, key_bias_d=None):
    """The compiled report's checks: finite, optimizer equivalence, and the device check. With
    attention present, a DEVICE_MISMATCH warning may only concern the key third of the
    projection bias (zero true gradient, see the module docstring)."""
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


def without_key_bias(name, values, key_bias_d):
    """A leaf's values with the attention key bias third removed (kept for every other leaf)."""
    values = np.asarray(values)
    if key_bias_d is not None and name.endswith("attn.qkv.b"):
        return np.concatenate([values[:key_bias_d], values[2 * key_bias_d:]])
    return values


def _leaves(tree):
    return [(name, leaf.numpy()) for name, leaf in rtree.paths(tree)]


def check_gradients(step, state, key_bias_d, device=DEVICE):
    """The first step's loss and every gradient leaf, device against oracle."""
    dev = rg.compile(step.loss_and_grads, (state,), validate="none", device=device)
    cpu = rg.compile(step.loss_and_grads, (state,), validate="none", device="cpu")
    (l1, g1), (l2, g2) = dev(state), cpu(state)
    assert abs(float(l1) - float(l2)) <= LOSS_TOL * abs(float(l2)), (float(l1), float(l2))
    worst = {}
    for (name, u), (_, v) in zip(_leaves(g1), _leaves(g2)):
        worst[name] = close_rel(without_key_bias(name, u, key_bias_d), without_key_bias(name, v, key_bias_d), GRAD_TOL, f"grad {name}")
    print("gradients: worst leaf", max(worst.items(), key=lambda kv: kv[1]), flush=True)
    return worst


def check_one_step(dev, cpu, step, state, key_bias_d):
    """One training step: loss, AdamW moments per leaf, and every parameter's update."""
    (s1, l1), (s2, l2) = dev(state), cpu(state)
    assert abs(float(l1) - float(l2)) <= LOSS_TOL * abs(float(l2)), (float(l1), float(l2))
    moments, updates = {}, {}
    for part in ("mu", "nu"):
        for (name, u), (_, v) in zip(_leaves(s1["opt"][part]), _leaves(s2["opt"][part])):
            moments[f"{part}.{name}"] = close_rel(without_key_bias(name, u, key_bias_d), without_key_bias(name, v, key_bias_d),
                                                  GRAD_TOL, f"{part} {name}")
    count1, count2 = float(s1["opt"]["count"]), float(s2["opt"]["count"])
    rows = zip(_leaves(state["params"]), _leaves(s1["params"]), _leaves(s2["params"]), _leaves(s1["opt"]["mu"]),
               _leaves(s2["opt"]["mu"]), _leaves(s1["opt"]["nu"]), _leaves(s2["opt"]["nu"]))
    for (name, p0), (_, p1), (_, p2), (_, m1), (_, m2), (_, v1), (_, v2) in rows:
        cut = lambda x: without_key_bias(name, x, key_bias_d)
        updates[name] = updates_agree(cut(p0), (cut(p1), cut(m1), cut(v1), count1), (cut(p2), cut(m2), cut(v2), count2),
                                      GRAD_TOL, name, step.adamw)
    print("one step: worst moment", max(moments.items(), key=lambda kv: kv[1]),
          "worst update residual", max(updates.items(), key=lambda kv: kv[1]), flush=True)
    return moments, updates


def check_run(dev, cpu, state, steps, key_bias_d):
    """`steps` device-loop steps: per-step losses, and each parameter's movement per leaf."""
    a = rg.run(dev, state, steps=steps)
    b = rg.run(cpu, state, steps=steps)
    assert a.status == b.status == "completed"
    la, lb = np.array(a.history["aux"], np.float64), np.array(b.history["aux"], np.float64)
    rel = np.abs(la - lb) / np.abs(lb)
    assert rel.max() <= LOSS_TOL, (int(np.argmax(rel)), la, lb)
    movement = {}
    for (name, p0), (_, p1), (_, p2) in zip(_leaves(state["params"]), _leaves(a.state["params"]), _leaves(b.state["params"])):
        cut = lambda x: without_key_bias(name, np.asarray(x, np.float64), key_bias_d)
        d1, d2 = cut(p1) - cut(p0), cut(p2) - cut(p0)
        norm = float(np.linalg.norm(d2))
        movement[name] = float(np.linalg.norm(d1 - d2)) / norm if norm > 0 else float(np.linalg.norm(d1))
        assert movement[name] <= MOVE_TOL, (f"movement of {name} over {steps} steps", movement[name])
    print(f"{steps} steps: loss worst {rel.max():.2e}, worst movement", max(movement.items(), key=lambda kv: kv[1]), flush=True)
    return rel.max(), movement


def full_check(step, state, steps, key_bias_d=None, device=DEVICE, standard=True):
    print(f"compile for {device} and cpu, {steps} steps", flush=True)
    dev = rg.compile(step, (state,), validate="standard" if standard else "none", device=device)
    cpu = rg.compile(step, (state,), validate="none", device="cpu")
    if standard:
        _device_check(dev, key_bias_d)
    check_gradients(step, state, key_bias_d, device)
    check_one_step(dev, cpu, step, state, key_bias_d)
    check_run(dev, cpu, state, steps, key_bias_d)


def test_c2_mlp_full_size():
    """C2: 4096 x 512 -> 2048 -> 2048 -> 1, gelu, AdamW; x drawn in-graph each step."""
    step, state = workloads.mlp_train_step(workloads.MLPConfig())
    full_check(step, state, 3)


@pytest.mark.parametrize("name,steps", [("C3", 3), ("C4", 2)])
def test_gpt_full_size(name, steps):
    """C3 (tied embeddings) and C4 (the headline) at full size."""
    cfg = workloads.GPT_CONFIGS[name]
    step, state = workloads.gpt_train_step(cfg)
    full_check(step, state, steps, key_bias_d=cfg.d)


def test_c5_matrix_chain_full_size():
    """C5: sum(((A@B)@C)@D) and its gradients for B and C; n = 4096, k = 8."""
    program, inputs = workloads.matrix_chain()
    gpu = rg.compile(program, inputs, validate="standard", device="hip")
    _device_check(gpu)
    cpu = rg.compile(program, inputs, validate="none", device="cpu")
    (value, gb, gc), (cv, cb, cc) = gpu(*inputs), cpu(*inputs)
    for name, u, v in (("dB", gb, cb), ("dC", gc, cc)):
        close_rel(u.numpy(), v.numpy(), GRAD_TOL, name)
    # The value sums 64 cancelling products of 4096-term chains: compare it against the sum of
    # the magnitudes it cancels, |A@B@C| @ |D| summed, which bounds every ordering's error.
    a, b, c, d = (x.numpy().astype(np.float64) for x in inputs)
    magnitude = float((np.abs(a @ b @ c) @ np.abs(d)).sum())
    assert abs(float(value) - float(cv)) <= 1e-6 * magnitude, (float(value), float(cv), magnitude)
