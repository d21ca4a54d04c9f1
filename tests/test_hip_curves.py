"""Full-length training runs on the HIP device overlaid on the CPU oracle's committed curves.

tests/golden/loss_curves.json holds the oracle's per-step losses for C2 (all 200 steps), C3
(all 300) and C4 (all 300), written by tests/golden/make_loss_curves.py, and summaries of each
parameter's movement over the run. Each test runs the whole device loop once (`rg.run`, no Python
between steps) and compares every step.

Tolerances:
- loss, every step: 1e-5 relative. The device sums in other orders (MFMA tiles, split-K, wave
  reductions), so its losses are not the oracle's bits; the largest per-step difference seen
  over the full runs on an MI355X is 5.2e-7 (C2, C3 and C4 alike; each run prints its own).
- movement, per parameter leaf: d = final - initial against the fixture's summaries of the
  oracle's d: its L2 norm within MOVE_TOL = 1e-4 relative, and its dot products with PROJECTIONS
  fixed random vectors within 4.5 * MOVE_TOL * |d_oracle|. Largest seen on an MI355X over the
  full runs: norm 5.1e-6 (C2), 2.5e-6 (C3), 2.1e-6 (C4); projection 6.1e-6 (C2), 1.2e-4 (C3, a
  query-key-value weight), 4.1e-5 (C4), each relative to |d_oracle|. For a device movement d', the projection
  difference (d' - d) . r is normal with deviation |d' - d|, so the projections bound the
  movement's L2 error without storing the parameters (4.5 deviations: over ~300 leaf and
  projection pairs a chance failure has probability under 0.3 %). The final state itself is
  not compared: it is dominated by the initial weights. The attention projection bias's key
  third is left out: its true gradient is exactly zero (softmax ignores a per-row shift of the
  scores), so both sides hold rounding noise that AdamW scales up to the learning rate; its q
  and v thirds are compared.
"""

import importlib.util
import json
import os

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import workloads

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "loss_curves.json")
LOSS_TOL = 1e-5
MOVE_TOL = 1e-4


def _generator():
    """tests/golden/make_loss_curves.py, for its projection vectors."""
    spec = importlib.util.spec_from_file_location("make_loss_curves", os.path.join(os.path.dirname(FIXTURE), "make_loss_curves.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _fixture(name):
    with open(FIXTURE) as f:
        return json.load(f)[name]


@pytest.mark.parametrize("name", ["C2", "C3", "C4"])
def test_full_length_loss_curve_overlays_the_oracle(name):
    fx = _fixture(name)
    if name == "C2":
        step, state = workloads.mlp_train_step()
    else:
        step, state = workloads.gpt_train_step(workloads.GPT_CONFIGS[name])
    print(f"{name}: compile for hip, run {fx['steps']} steps", flush=True)
    c = rg.compile(step, (state,), validate="none", device="hip")
    r = rg.run(c, state, steps=fx["steps"])
    assert r.status == "completed" and r.steps == fx["steps"], r
    got, want = np.array(r.history["aux"]), np.array(fx["loss"])
    rel = np.abs(got - want) / np.abs(want)
    worst = int(np.argmax(rel))
    print(f"{name}: largest relative loss difference {rel.max():.3e} at step {worst} "
          f"(hip {got[worst]!r}, oracle {want[worst]!r}); mean {rel.mean():.3e}", flush=True)
    assert rel.max() <= LOSS_TOL, f"step {worst}: hip {got[worst]} oracle {want[worst]}"

    gen = _generator()
    mine = gen.movement_stats(state["params"], r.state["params"])
    assert set(mine) == set(fx["movement"]), set(mine) ^ set(fx["movement"])
    errors = {}
    for leaf, ref in fx["movement"].items():
        if leaf.endswith("attn.qkv.b[k]") or ref["norm"] == 0.0:
            continue
        got_leaf = mine[leaf]
        norm_err = abs(got_leaf["norm"] - ref["norm"]) / ref["norm"]
        proj_err = max(abs(a - b) for a, b in zip(got_leaf["proj"], ref["proj"])) / ref["norm"]
        errors[leaf] = (norm_err, proj_err)
        assert norm_err <= MOVE_TOL and proj_err <= 4.5 * MOVE_TOL, (leaf, norm_err, proj_err)
    worst_norm = max(errors.items(), key=lambda kv: kv[1][0])
    worst_proj = max(errors.items(), key=lambda kv: kv[1][1])
    print(f"{name}: movement norm worst {worst_norm}, projection worst {worst_proj}", flush=True)
