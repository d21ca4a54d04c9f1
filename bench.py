"""Headline benchmark: train steps/s of the d=256, 6-layer char-GPT on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline | --cpu-full]

One step is one full AdamW training step of the C4 program (B=32, T=256, d=256, 8 heads, 6 layers,
vocab 96, fp32): ids drawn in the step from the state key, forward, backward, update. The timed
region is `rg.run(compiled, state, steps=K)`: the device-resident step loop, synchronized on
both sides. Prints one JSON line with the throughput, the roofline of the dominant kernel class
(each class's device time inside the pass: every plan step replayed back to back between HIP
events on the execution stream, minus the same replay without the class's steps), and the CPU
oracle's time for steps of the same program on this host as the baseline.
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
FP32_MFMA_PEAK_TFLOPS = 157.3


def _numel(s):
    n = 1
    for d in s:
        n *= d
    return n


def classify(plan, runs_in=None):
    """Groups plan steps into kernel classes with their algorithmic work and the step indices of
    each. The work of a step is the engine's (plan_summary's flops, bytes and bound): flops for
    attention and for products on matrix cores, bytes (each distinct input read once, each
    output written once) for everything else, including the products the backend streams.

    `runs_in` (Compiled step_runs_in) names, per step, the step whose kernel computes it. The
    steps one kernel computes form one unit: products only (a grouped launch) stay in their class
    with their flops, counted as one launch; a product with the elementwise group of its epilogue
    (and a column sum of that group's output) forms the class `gemm_mfma_epilogue`: the product's
    flops, the other steps' bytes beside the product's, one launch, so the combined kernel's time
    is neither charged to the plain products nor counted as elementwise work done in no time; an
    attention backward with the column sum it computes stays in `attention`, the sum's bytes
    beside its flops."""
    classes = {}
    runs_in = runs_in or list(range(len(plan)))
    members = {}
    for k, r in enumerate(runs_in):
        members.setdefault(r, []).append(k)

    def add(name, k, st, launch=True):
        c = classes.setdefault(name, {"steps": [], "flops": 0.0, "executed_flops": 0.0, "bytes": 0.0, "launches": 0})
        c["steps"].append(k)
        if st["bound"] == "mfma":
            c["flops"] += st["flops"]
            c["executed_flops"] += st.get("executed_flops", st["flops"])
        c["bytes"] += st["bytes"]
        c["launches"] += 1 if launch else 0

    def is_product(q):
        return plan[q]["kind"] == "instr" and plan[q].get("op") in ("matmul", "matmul_t")

    for k, st in enumerate(plan):
        unit = members[runs_in[k]]
        combined = len(unit) > 1
        products_only = combined and all(is_product(q) for q in unit)
        launch = runs_in[k] == k
        if combined and not products_only:
            attn = any(plan[q]["kind"] == "attention" for q in unit)
            main = st["kind"] == "attention" if attn else is_product(k)
            add("attention" if attn else "gemm_mfma_epilogue", k, st if main else dict(st, bound="hbm"), launch=launch)
        elif st["kind"] == "attention":
            add("attention", k, st)
        elif st["kind"] == "fused":
            add("fused_elementwise", k, st)
        elif st["op"] in ("matmul", "matmul_t"):
            shape = st["shape"]
            n_cols = shape[-1] if shape else 1
            m_rows = _numel(shape) // max(n_cols, 1)
            if st["bound"] != "mfma":
                add("gemm_skinny", k, st, launch=launch)
            else:
                add("gemm_mfma" if len(shape) >= 2 and n_cols >= 32 and m_rows >= 32 else "gemm_plain", k, st, launch=launch)
        elif st["op"] in ("sum", "max", "min"):
            add("reduce", k, st)
        elif st["op"] in ("take", "take_along", "take_grad", "take_along_grad"):
            add("gather_scatter", k, st)
        else:
            add("structural_other", k, st)
    return classes


def time_classes(compiled, inputs, classes, repeats, trials=15):
    """Device seconds per pass of each kernel class, measured inside the pass: every plan step
    replayed back to back `repeats` times between two HIP events on the execution stream, minus
    the same replay without the class's steps, timed right after it (rg_hip_exec_time_steps);
    the median over `trials` such pairs, so that a slow drift of the clock cancels. The class's
    kernels so run with the caches and clocks they meet inside a training step (the operands a
    product or attention step reads were just written by the step before it), and no event
    separates them. The replay of the class's steps alone is kept as `isolated_seconds`.
    Returns the seconds of the whole replayed pass."""
    def once(steps):
        return compiled._n.time_steps(inputs, steps, repeats) / repeats if steps else 0.0

    def median(xs):
        return sorted(xs)[len(xs) // 2]

    every = sorted(s for c in classes.values() for s in c["steps"])
    fulls = []
    for c in classes.values():
        own = set(c["steps"])
        rest = [s for s in every if s not in own]
        diffs = []
        for _ in range(trials):
            f = once(every)
            fulls.append(f)
            diffs.append(f - once(rest))
        in_pass = median(diffs)
        c["isolated_seconds"] = median([once(c["steps"]) for _ in range(trials)])
        # A class too small to stand out of the pass's run-to-run spread (its difference of two
        # passes under half or over twice its time replayed alone) keeps its isolated time.
        iso = c["isolated_seconds"]
        c["timing"] = "in_pass" if 0.5 * iso <= in_pass <= 2.0 * iso else "isolated"
        c["seconds"] = in_pass if c["timing"] == "in_pass" else c["isolated_seconds"]
        if c["flops"]:
            c["achieved"], c["unit"] = c["flops"] / c["seconds"] / 1e12, "TFLOP/s"
        else:
            c["achieved"], c["unit"] = c["bytes"] / c["seconds"] / 1e9, "GB/s"
    return median(fulls)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c4_hbm_traffic.txt")


def measured_traffic(workload, kernel_class):
    """HBM bytes per launch of `kernel_class`, from the counter summary committed under profiles/
    (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this script on C4, scaled by the copy-kernel
    calibration recorded in the same file), or None when no measurement exists (any other workload)."""
    if workload != "C4":
        return None
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel_class:
                    return int(float(parts[2]))
    except OSError:
        pass
    return None


def copy_probe(rg):
    """A plain copy kernel of known size, for calibrating the FETCH_SIZE/WRITE_SIZE counters:
    y = -x over 64 Mi fp32 elements (256 MiB read, 256 MiB written per launch), 10 launches."""
    import numpy as np
    n = 64 << 20
    x = rg.tensor(np.ones(n, np.float32))
    c = rg.compile(lambda x: -x, (x,), validate="none", device="hip")
    for _ in range(10):
        c(x)
    print(json.dumps({"probe": "copy", "elements": n, "bytes_read_per_launch": 4 * n, "bytes_written_per_launch": 4 * n,
                      "launches": 10}), flush=True)


def cpu_baseline(cfg, sample_batch=4, steps=3):
    """The CPU oracle (a restatement of rg's CPU interpreter) on the same workload: one warm-up
    step and `steps` timed steps (BASELINE's 1 + 3-5). A full C4 step takes about a minute on the
    host, so by default the steps run the same model at `sample_batch` of its sequences and the
    rate is extrapolated to the full batch (`extrapolated` true, the measured sample time beside
    it): the cost is proportional to the tokens in the batch (the products' row counts and
    attention are per sequence), except the optimizer update, whose fixed cost the scaling counts
    `batch / sample_batch` times, so the estimate errs towards a slower CPU. `sample_batch` equal
    to the batch (bench.py --cpu-full) times the full workload itself."""
    from rustautograd_amd import _native, workloads
    import rustautograd_amd as rg
    import ctypes
    path = os.path.join(ROOT, "oracle", "_build", "librg_cpu.so")
    _native.register_backend("cpu", path, "rg_cpu_")
    threads = ctypes.CDLL(path).rg_cpu_threads()
    sample = cfg._replace(batch=min(sample_batch, cfg.batch))
    step, state = workloads.gpt_train_step(sample)
    c = rg.compile(step, (state,), validate="none", device="cpu")
    warm = rg.run(c, state, steps=1)
    r = rg.run(c, warm.state, steps=steps)
    per_step = r.elapsed / r.steps
    scale = sample.batch / cfg.batch
    full = sample.batch == cfg.batch
    how = (f"1 warm-up + {r.steps} timed AdamW steps of the full workload (batch {cfg.batch}, T={cfg.block})" if full else
           f"1 warm-up + {r.steps} timed AdamW steps of the same model at batch {sample.batch} of {cfg.batch} (T={cfg.block}), "
           f"steps/s scaled by {sample.batch}/{cfg.batch}")
    return {"value": 1.0 / per_step * scale, "unit": "steps/s", "cores": int(threads), "kind": "port",
            "extrapolated": not full, "sample_batch": sample.batch, "sample_seconds_per_step": round(per_step, 3),
            "sample": f"{how}, on the oracle (oracle/cpu_exec.cpp): {per_step:.2f} s per measured step; OpenMP threads where the "
                      f"reference uses rayon"}


def roofline_of(compiled, inputs, reps, workload):
    """(roofline dict, per-class table, device seconds per pass) from each kernel class's device
    time inside the replayed pass (time_classes)."""
    runs_in = compiled._n.step_runs_in() if hasattr(compiled._n, "step_runs_in") else None
    classes = classify(compiled.plan_summary(), runs_in)
    time_classes(compiled, inputs, classes, 1, trials=1)
    total_s = time_classes(compiled, inputs, classes, reps)
    dom_name, dom = max(classes.items(), key=lambda kv: kv[1]["seconds"])
    per_launch = (dom["flops"] or dom["bytes"]) / dom["launches"]
    # The dominant class's launches timed alone (its steps replayed back to back between two HIP
    # events on the execution stream): the per-launch duration a kernel trace reports. The
    # in-pass figure (the pass minus the pass without the class) also credits the overlap of
    # each launch's start with the end of the kernel before it; it is kept beside.
    avg_s = dom["isolated_seconds"] / dom["launches"]
    achieved = per_launch / avg_s / (1e12 if dom["flops"] else 1e9)
    if dom["flops"]:
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roof["traffic"] = measured_traffic(workload, dom_name)
    roof.update({"kernel": dom_name, "launches_per_step": dom["launches"], "algorithmic_per_launch": round(per_launch),
                 "algorithmic_bytes_per_launch": round(dom["bytes"] / dom["launches"]), "avg_launch_us": round(avg_s * 1e6, 2),
                 "in_pass_avg_launch_us": round(dom["seconds"] / dom["launches"] * 1e6, 2)})
    kernels = {k: {"ms_per_step": round(v["seconds"] * 1e3, 3), "launches": v["launches"], "achieved": round(v["achieved"], 2),
                   "unit": v["unit"], "frac": round(v["achieved"] / (FP32_MFMA_PEAK_TFLOPS if v["unit"] == "TFLOP/s" else HBM_PEAK_GBS), 4),
                   "isolated_ms_per_step": round(v["isolated_seconds"] * 1e3, 3), "timing": v["timing"]}
               for k, v in sorted(classes.items(), key=lambda kv: -kv[1]["seconds"])}
    for k, v in classes.items():
        # Attention skips the tiles a constant mask hides: its rate over the products it executes
        # beside the rate over all the products of the unfused graph it replaces.
        if v["flops"] and v["executed_flops"] != v["flops"]:
            ex = v["executed_flops"] / v["seconds"] / 1e12
            kernels[k].update({"executed_share": round(v["executed_flops"] / v["flops"], 5), "executed_achieved": round(ex, 2),
                               "executed_frac": round(ex / FP32_MFMA_PEAK_TFLOPS, 4)})
    return roof, kernels, total_s


def bench_program(args, rg, workloads):
    """C5: one evaluation of the matrix-chain program (value and the gradients for B and C) per
    pass. Timed region: `repeats` back-to-back passes over the whole plan between two HIP events,
    the inputs already in HBM (rg_hip_exec_time_steps)."""
    program, inputs = workloads.matrix_chain()
    compiled = rg.compile(program, inputs, validate="basic", device="hip")
    natives = [x._t for x in inputs]
    every = list(range(len(compiled.plan_summary())))
    compiled._n.time_steps(natives, every, max(1, args.warmup))
    passes = max(1, args.steps)
    seconds = [compiled._n.time_steps(natives, every, passes) for _ in range(max(1, args.repeats))]
    sec = sorted(seconds)[len(seconds) // 2]
    value = passes / sec
    print(f"# C5: {passes} passes in {sec * 1e3:.3f} ms (median of {len(seconds)})", file=sys.stderr, flush=True)
    roof, kernels, total_s = roofline_of(compiled, natives, max(1, args.timing_reps), "C5")
    n, k = 4096, 8
    # The reordered plan reads B once and C twice (A@B, then (A@B)@C and the gradient through C)
    # and writes dB and dC: five n x n fp32 matrices; the k-wide operands are noise beside them.
    moved = 5 * n * n * 4
    return {
        "metric": "C5 matrix-chain passes/s (value + dB + dC) on 1 MI355X; % of HBM roofline",
        "value": round(value, 2), "unit": "passes/s", "n_gpus": 1, "steps": passes, "warmup": args.warmup,
        "ms_per_step": round(1e3 / value, 4),
        "timed_region": "back-to-back replays of every plan step between two HIP events, inputs resident in HBM; median of repeats",
        "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: A, B, C, D ~ N(0, 1/64) from numpy default_rng(0)",
        "config": {"workload": "C5 matrix chain sum(((A@B)@C)@D), gradients w.r.t. B and C, e-graph reordered plan",
                   "n": n, "k": k, "gflop_per_pass": 1.34, "min_hbm_mb_per_pass": round(moved / 1e6, 1)},
        "roofline": roof, "kernels": kernels, "device_ms_per_step": round(total_s * 1e3, 4),
        "pass_hbm_fraction": round(moved / (1e3 / value * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "cpu_baseline": None,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--repeats", type=int, default=3, help="timed runs of K steps; the median is reported")
    ap.add_argument("--workload", default="C4", choices=["C2", "C3", "C4", "C5"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-full", action="store_true",
                    help="time the CPU baseline on the full batch (1 warm-up + 3 steps, several minutes) instead of extrapolating")
    ap.add_argument("--timing-reps", type=int, default=5, help="per-step HIP-event timing passes after the timed run (0: skip)")
    ap.add_argument("--probe", choices=["copy"], help="run only a plain copy kernel of known size (for counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import rustautograd_amd as rg
    from rustautograd_amd import _native, workloads
    if "hip" not in rg.devices():
        raise SystemExit(f"HIP backend unavailable: {_native.hip_error()}")
    if args.probe == "copy":
        copy_probe(rg)
        return
    if args.workload == "C5":
        print(json.dumps(bench_program(args, rg, workloads)), flush=True)
        return
    if args.workload == "C2":
        cfg = workloads.MLPConfig()
        step, state = workloads.mlp_train_step(cfg)
    else:
        cfg = workloads.GPT_CONFIGS[args.workload]
        step, state = workloads.gpt_train_step(cfg)
    t0 = time.perf_counter()
    compiled = rg.compile(step, (state,), validate="basic", device="hip")
    compile_s = time.perf_counter() - t0
    print(f"# compiled {args.workload} in {compile_s:.1f}s: {compiled.report['graph']['steps']} plan steps, "
          f"{compiled.report['graph']['fused_groups']} fused groups", file=sys.stderr, flush=True)

    warm = rg.run(compiled, state, steps=args.warmup) if args.warmup else None
    cur = warm.state if warm else state
    # The timed region is the step loop of `rg.run` (RunOut.seconds, reference validate.rs:264-265,
    # 322-360): K steps on the device with the state already in HBM, bracketed by a device
    # synchronization on both sides inside rg_hip_exec_run. The median of `repeats` runs is
    # reported, as the reference's benches/gpt_compare.py:48-53 does. The wall time of the whole
    # rg.run call (state upload and final read over PCIe included) is reported beside it.
    loops, walls = [], []
    for _ in range(max(1, args.repeats)):
        t0 = time.perf_counter()
        res = rg.run(compiled, cur, steps=args.steps)
        walls.append(time.perf_counter() - t0)
        assert res.steps == args.steps, res
        loops.append(res.elapsed)
    loop_s, wall_s = sorted(loops)[len(loops) // 2], sorted(walls)[len(walls) // 2]
    value = args.steps / loop_s
    print(f"# {args.steps} steps: step loop {loop_s:.4f}s (median of {len(loops)}: {', '.join(f'{x:.4f}' for x in loops)}), "
          f"whole rg.run {wall_s:.4f}s; loss {res.history['aux'][0]:.4f} -> {res.history['aux'][-1]:.4f}", file=sys.stderr, flush=True)

    roof, kernels, total_s = None, None, None
    if args.timing_reps > 0:
        inputs = [rg.tensor(x)._t for x in rg.tree.leaves((res.state,))]
        roof, kernels, total_s = roofline_of(compiled, inputs, args.timing_reps, args.workload)

    if args.workload == "C2":
        metric = "train steps/s, MLP 512-2048-2048-1 batch 4096 (C2) on 1 MI355X; % of HBM / fp32-MFMA roofline"
        data = "synthetic: x ~ N(0,1) drawn inside the step from a seeded key, target sum(sin(x[:, :16])); random-init weights"
        config = {"workload": "C2 MLP regression training step", "batch": cfg.batch, "d_in": cfg.d_in, "hidden": cfg.hidden,
                  "optimizer": "adamw", "lr": cfg.lr, "gemm_gflop_per_step": 120.3}
        cpu = None
    else:
        metric = "train steps/s, char-GPT d=256 6L on 1 MI355X; % of HBM / fp32-MFMA roofline"
        if args.workload != "C4":
            metric = f"train steps/s, char-GPT {args.workload} on 1 MI355X; % of HBM / fp32-MFMA roofline"
        data = "synthetic: token ids uniform in [0,96) drawn inside the step from a seeded key; random-init weights"
        config = {"workload": f"{args.workload} char-GPT training step", "batch": cfg.batch, "seq_len": cfg.block, "d_model": cfg.d,
                  "heads": cfg.heads, "layers": cfg.layers, "vocab": cfg.vocab, "optimizer": "adamw", "lr": cfg.lr,
                  "gemm_gflop_per_step": round(workloads.gpt_gemm_flops(cfg) / 1e9, 2)}
        cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, sample_batch=cfg.batch if args.cpu_full else 4)
    out = {
        "metric": metric,
        "value": round(value, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 / value, 3),
        "timed_region": "rg.run step loop: K steps on the device, state resident in HBM, device-synchronized on both sides; median of repeats",
        "whole_run_steps_per_s": round(args.steps / wall_s, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": data,
        "config": config,
        "roofline": roof,
        "kernels": kernels,
        "device_ms_per_step": round(total_s * 1e3, 3) if total_s else None,
        "cpu_baseline": cpu,
    }
    if cpu:
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
