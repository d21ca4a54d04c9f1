"""Writes tests/golden/loss_curves.json: the CPU oracle's per-step training losses for the
BASELINE configurations C2 (200 steps), C3 (300 steps) and C4 (300 steps), summary statistics
of every state leaf after the last step, and of every parameter's movement over the run.

    python tests/golden/make_loss_curves.py [C2 C3 C4]

The oracle (oracle/cpu_exec.cpp, a restatement of the reference's CPU interpreter) runs the
same programs the device tests compile (rustautograd_amd/workloads.py), on the reference's CPU
plan (Fuse::DEFAULT), with its checker-only row-parallel products, which are bit-identical to
the reference's serial loop (tests/test_engine.py checks that). The device tests overlay their
own full runs on these curves. CPU only; takes about an hour on 8 cores (C4 is 8 s a step).

Movement summaries: for each parameter leaf, d = final - initial in float64, its L2 norm and
its dot products with PROJECTIONS fixed random vectors (`projection(n, k)`, standard normal
from seed 1000 + k). For a device run with movement d', (d' - d) . r has standard deviation
|d' - d|, so the projections' differences measure the device's movement error in the L2 norm
without storing the parameters.
"""

import ctypes
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

STEPS = {"C2": 200, "C3": 300, "C4": 300}
PROJECTIONS = 4
OUT = os.path.join(HERE, "loss_curves.json")


def _summary(v):
    return {"n": int(v.size), "sum": float(v.sum()), "sumsq": float((v * v).sum()), "absmax": float(np.abs(v).max()) if v.size else 0.0}


def leaf_stats(state):
    """Sum, sum of squares and largest magnitude of every state leaf (float64). The attention
    projection bias is summarized per third (q, k, v): the key third has a zero true gradient,
    so its values are rounding noise scaled by AdamW, and the device tests leave it out."""
    import rustautograd_amd as rg
    stats = {}
    for name, leaf in rg.tree.paths(state):
        v = leaf.numpy().astype(np.float64)
        if name.endswith("attn.qkv.b"):
            for part, third in zip("qkv", np.split(v, 3)):
                stats[f"{name}[{part}]"] = _summary(third)
        else:
            stats[name] = _summary(v)
    return stats


def projection(n, k):
    """The k-th fixed random vector of length n the movement summaries project onto."""
    return np.random.default_rng(1000 + k).standard_normal(n)


def _split_key_bias(name, v):
    if name.endswith("attn.qkv.b"):
        return [(f"{name}[{part}]", third) for part, third in zip("qkv", np.split(v, 3))]
    return [(name, v)]


def movement_stats(initial, final):
    """Per parameter leaf (the attention projection bias per third): the L2 norm of final -
    initial and its projections on the fixed random vectors."""
    import rustautograd_amd as rg
    stats = {}
    for (name, a), (_, b) in zip(rg.tree.paths(initial), rg.tree.paths(final)):
        d = b.numpy().astype(np.float64).ravel() - a.numpy().astype(np.float64).ravel()
        for leaf, part in _split_key_bias(name, d):
            stats[leaf] = {"norm": float(np.linalg.norm(part)),
                           "proj": [float(part @ projection(part.size, k)) for k in range(PROJECTIONS)]}
    return stats


def main(which):
    import rustautograd_amd as rg
    from rustautograd_amd import _native, workloads
    oracle = os.path.join(ROOT, "oracle", "_build", "librg_cpu.so")
    _native.register_backend("cpu", oracle, "rg_cpu_")
    ctypes.CDLL(oracle).rg_cpu_set_row_parallel_gemm(1)
    data = json.load(open(OUT)) if os.path.exists(OUT) else {}
    for name in which:
        step, state = workloads.mlp_train_step() if name == "C2" else workloads.gpt_train_step(workloads.GPT_CONFIGS[name])
        c = rg.compile(step, (state,), validate="none", device="cpu")
        t0 = time.time()
        r = rg.run(c, state, steps=STEPS[name])
        assert r.status == "completed", r
        data[name] = {
            "steps": r.steps,
            "loss": [float(x) for x in r.history["aux"]],
            "final_state": leaf_stats(r.state),
            "movement": movement_stats(state["params"], r.state["params"]),
            "oracle_seconds": round(time.time() - t0, 1),
        }
        print(f"{name}: {r.steps} steps in {time.time() - t0:.0f}s, loss {r.history['aux'][0]:.6f} -> {r.history['aux'][-1]:.6f}",
              flush=True)
        with open(OUT, "w") as f:
            json.dump(data, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1:] or list(STEPS))
