"""Compiled programs on the HIP device against the CPU oracle: the run loop, state handoff,
pooled frames, failure latching and the benchmark programs (tests/metal.rs:248-390 and
test_framework.py:447-473 of the reference)."""

import ctypes

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import _rg, nn, optim, random, workloads

from helpers import RunDesc, RunResult, close, hip_abi, hip_program, op, seq, t

pytestmark = pytest.mark.gpu


def _gd_graph():
    g = _rg.Graph()
    w, x, y = g.input([3], "float32"), g.input([8, 3], "float32"), g.input([8], "float32")
    p = op(g, "matmul", [x, w])
    e = op(g, "sub", [p, y])
    sq = op(g, "mul", [e, e])
    l = op(g, "sum", [sq], axes=[0], keepdims=False)
    gr = g.grad(l, [w])[0]
    lr = g.constant(rg.tensor(np.float32(0.01))._t)
    nw = op(g, "sub", [w, op(g, "mul", [gr, lr])])
    return g, [nw, l]


def test_run_loop_trains_on_the_device_and_matches_cpu():
    g, outs = _gd_graph()
    inputs = [t(np.zeros(3)), seq((8, 3)), t(np.arange(1, 9))]
    gpu = _rg.compile(g, outs, [x._t for x in inputs], "standard", "hip", "standard")
    cpu = _rg.compile(g, outs, [x._t for x in inputs], "standard", "cpu", "standard")
    import json
    rep = json.loads(gpu.report_json)
    assert rep["status"] == "ok", rep
    assert rep["device"] == "hip"
    assert {c["name"]: c["status"] for c in rep["checks"]}["device_equivalence"] == "pass"
    batch = [[inputs[1]._t, inputs[2]._t]]
    a = gpu.run([(0, 0)], [1, 2], [1], [inputs[0]._t], batch, 200)
    b = cpu.run([(0, 0)], [1, 2], [1], [inputs[0]._t], batch, 200)
    assert a[3] == 200
    close(rg.Tensor(a[0][0]).numpy(), rg.Tensor(b[0][0]).numpy(), 1e-3, "state after 200 steps")
    assert a[2][0][199] < a[2][0][0]
    close(np.array(a[2][0]), np.array(b[2][0]), 1e-4, "loss history")


def test_device_loop_equals_stepping_one_at_a_time():
    g, outs = _gd_graph()
    inputs = [t(np.zeros(3)), seq((8, 3)), t(np.arange(1, 9))]
    c = _rg.compile(g, outs, [x._t for x in inputs], "basic", "hip", "standard")
    batch = [[inputs[1]._t, inputs[2]._t]]
    many = c.run([(0, 0)], [1, 2], [1], [inputs[0]._t], batch, 7)
    state = [inputs[0]._t]
    hist = []
    for _ in range(7):
        one = c.run([(0, 0)], [1, 2], [1], state, batch, 1)
        state = one[0]
        hist += one[2][0]
    assert np.array_equal(rg.Tensor(many[0][0]).numpy(), rg.Tensor(state[0]).numpy())
    assert many[2][0] == hist


def test_batches_cycle_on_the_device():
    g, outs = _gd_graph()
    inputs = [t(np.zeros(3)), seq((8, 3)), t(np.arange(1, 9))]
    b2 = [t(np.asarray(inputs[1].numpy()) * 0.5)._t, t(np.arange(8, 0, -1))._t]
    batches = [[inputs[1]._t, inputs[2]._t], b2]
    gpu = _rg.compile(g, outs, [x._t for x in inputs], "basic", "hip", "standard")
    cpu = _rg.compile(g, outs, [x._t for x in inputs], "basic", "cpu", "standard")
    a = gpu.run([(0, 0)], [1, 2], [1], [inputs[0]._t], batches, 9)
    b = cpu.run([(0, 0)], [1, 2], [1], [inputs[0]._t], batches, 9)
    close(np.array(a[2][0]), np.array(b[2][0]), 1e-5, "cycled history")


def test_swapped_state_and_pooled_frames_keep_constants():
    def step(w):
        return rg.tanh(w) + w
    x = seq((512,))
    gpu = rg.compile(step, (x,), validate="basic", device="hip")
    cpu = rg.compile(step, (x,), validate="basic", device="cpu")
    close(rg.run(gpu, x, steps=50).state.numpy(), rg.run(cpu, x, steps=50).state.numpy(), 1e-4, "swapped state")

    c = rg.compile(lambda w: w * rg.tensor([1.0, 2.0, 3.0, 4.0]), (rg.ones(4),), validate="basic", device="hip")
    first = rg.run(c, rg.ones(4), steps=3).state.numpy()
    for _ in range(4):
        assert np.array_equal(rg.run(c, rg.ones(4), steps=3).state.numpy(), first)
    assert first.tolist() == [1.0, 8.0, 27.0, 64.0]


def test_nonfinite_stop_matches_the_host_loop():
    def step(w):
        w2 = w * 3.0
        return w2, w2.sum()
    x = t([1e30, 1.0])
    gpu = rg.compile(step, (x,), validate="basic", device="hip")
    cpu = rg.compile(step, (x,), validate="basic", device="cpu")
    a, b = rg.run(gpu, x, steps=100), rg.run(cpu, x, steps=100)
    assert a.status == b.status == "stopped_nonfinite"
    assert a.nonfinite_step == b.nonfinite_step
    assert a.steps == b.steps
    assert np.array_equal(a.state.numpy(), b.state.numpy())


def test_repeated_runs_do_not_leak_device_memory():
    """tests/metal.rs:278-301: frames come from the program's pool and the run loop's graphs and
    buffers stay with the frame, so 200 cycles of calls and runs hold no more device memory."""
    g = _rg.Graph()
    x = g.input([256, 256], "float32")
    y = op(g, "tanh", [op(g, "matmul", [x, x])])
    inp = seq((256, 256))
    c = _rg.compile(g, [y], [inp._t], "none", "hip", "none")

    def cycle():
        for _ in range(5):
            c.call([inp._t])
        c.run([(0, 0)], [], [], [inp._t], [], 5, True)
    cycle()
    before = c.allocated_bytes()
    for _ in range(200):
        cycle()
    after = c.allocated_bytes()
    assert after < before + 32 * 1024 * 1024, f"device memory grew from {before} to {after}"


def test_a_buffer_beyond_the_device_limit_is_refused_at_compile_time():
    """tests/metal.rs:354-363: a 16 TiB float32 value is refused when the program is built,
    before anything is allocated, as DEVICE_UNAVAILABLE naming the limit."""
    g = _rg.Graph()
    x = g.input([1], "float32")
    y = op(g, "tanh", [op(g, "broadcast_to", [x], shape=[1 << 42])])
    with pytest.raises(rg.DiagnosticError) as e:
        _rg.compile(g, [y], [t([0.5])._t], "none", "hip", "none")
    d = e.value.diagnostic
    assert d["code"] == "DEVICE_UNAVAILABLE", d
    assert "exceeds" in d["observation"]["detail"], d


def test_device_failure_reaches_the_caller_and_the_program_recovers():
    """tests/metal.rs:365-390: an injected failure surfaces as DEVICE_EXECUTION_FAILED from a
    call and from a run (with no completed steps), and the next run on a recycled frame is right."""
    x = t([1.0, 2.0, 3.0, 4.0])
    c = rg.compile(lambda w: w * 0.5, (x,), validate="basic", device="hip")
    c._n.inject_failure()
    with pytest.raises(rg.DiagnosticError) as e:
        c(x)
    d = e.value.diagnostic
    assert d["code"] == "DEVICE_EXECUTION_FAILED" and d["observation"]["detail"] == "injected failure", d
    c._n.inject_failure()
    with pytest.raises(rg.DiagnosticError) as e:
        rg.run(c, x, steps=10)
    d = e.value.diagnostic
    assert d["code"] == "DEVICE_EXECUTION_FAILED" and d["observation"]["completed_steps"] == 0, d
    assert d["observation"]["detail"] == "injected failure"
    ok = rg.run(c, x, steps=1)
    assert ok.status == "completed" and ok.state.numpy().tolist() == [0.5, 1.0, 1.5, 2.0]


def test_a_failure_in_the_middle_of_a_run_reports_the_completed_steps():
    """A failure after 5 of 10 steps reports 5 completed steps, with and without per-step history
    (the device loop runs in chunks with and without history), and the next run is right."""
    for with_aux in (False, True):
        def step(w):
            nw = w * 0.5
            return (nw, nw.sum()) if with_aux else nw
        x = t([1.0, 2.0, 3.0, 4.0])
        c = rg.compile(step, (x,), validate="basic", device="hip")
        c._n.inject_failure(after=5)
        with pytest.raises(rg.DiagnosticError) as e:
            rg.run(c, x, steps=10)
        d = e.value.diagnostic
        assert d["code"] == "DEVICE_EXECUTION_FAILED" and d["observation"]["completed_steps"] == 5, d
        r = rg.run(c, x, steps=3)
        assert r.state.numpy().tolist() == [0.125, 0.25, 0.375, 0.5]


def test_run_failure_leaves_the_state_of_the_completed_steps_at_the_abi():
    """Through the C ABI: after a failure the state slot holds the state after `done` steps (as
    the reference's host loop leaves it, validate.rs:329-335), not a half-run chunk."""
    lib = hip_abi()

    g = _rg.Graph()
    w = g.input([4], "float32")
    nw = op(g, "mul", [w, g.constant(rg.tensor(np.float32(0.5))._t)])
    prog, (win,), (wout, lout) = hip_program(lib, g, [nw, op(g, "sum", [nw], axes=[0], keepdims=False)])
    err = ctypes.create_string_buffer(4096)
    try:
        for history, fail_after in ((False, 5), (True, 70), (True, 0)):
            e = lib.rg_hip_exec_new(prog, err, len(err))
            assert e, err.value
            x0 = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
            assert lib.rg_hip_exec_write(e, win, x0.ctypes.data, 16) == 0
            swaps = (ctypes.c_int64 * 2)(win, wout)
            hs = (ctypes.c_int64 * 1)(lout)
            steps = 100
            hist = (ctypes.c_double * steps)()
            d = RunDesc(n_swaps=1, swaps=swaps, n_history=1 if history else 0, history_slots=hs, steps=steps, history=hist)
            lib.rg_hip_program_inject_failure_after(prog, fail_after)
            out = RunResult()
            assert lib.rg_hip_exec_run(e, ctypes.byref(d), ctypes.byref(out)) == -1
            assert out.done == fail_after, (history, out.done)
            msg = ctypes.create_string_buffer(256)
            assert lib.rg_hip_exec_failure(e, msg, 256) == 1 and msg.value == b"injected failure"
            got = np.zeros(4, np.float32)
            assert lib.rg_hip_exec_read(e, win, got.ctypes.data, 16) == 0
            assert np.array_equal(got, x0 * np.float32(0.5) ** fail_after), (history, got)
            lib.rg_hip_exec_free(e)
    finally:
        lib.rg_hip_program_free(prog)


def test_linear_regression_converges_and_matches_cpu():
    step, w0, batch = workloads.linreg()
    gpu = rg.compile(step, (w0, batch), validate="standard", device="hip")
    cpu = rg.compile(step, (w0, batch), validate="standard", device="cpu")
    assert gpu.report["status"] == "ok", gpu.report
    a, b = rg.run(gpu, w0, batch, steps=500), rg.run(cpu, w0, batch, steps=500)
    assert a.history["aux"][-1] < 1e-3
    close(np.array(a.history["aux"]), np.array(b.history["aux"]), 1e-4, "loss curve")
    close(a.state.numpy(), np.arange(8), 1e-3, "weights")


def test_small_gpt_loss_curve_overlays_cpu():
    cfg = workloads.GPT_CONFIGS["C3"]._replace(batch=4, block=32, layers=2)
    step, state = workloads.gpt_train_step(cfg)
    gpu = rg.compile(step, (state,), validate="standard", device="hip")
    cpu = rg.compile(step, (state,), validate="basic", device="cpu")
    assert gpu.report.ok, gpu.report["diagnostics"]
    checks = {c["name"]: c for c in gpu.report["checks"]}
    assert checks["finite"]["status"] == "pass" and checks["optimizer_equivalence"]["status"] == "pass"
    # The device check compares the state after one AdamW update. The attention key bias has a
    # mathematically zero gradient (softmax ignores a per-row shift of the scores), so its value is
    # rounding noise that Adam scales to +-lr; a DEVICE_MISMATCH may only point there.
    dev = checks["device_equivalence"]
    assert dev["detail"]["max_relative_error"] < 0.05, dev

    names = gpu._out_def.paths("out")
    for d in gpu.report["diagnostics"]:
        assert d["code"] == "DEVICE_MISMATCH", d
        name, element = names[d["observation"]["output_index"]], d["observation"]["element"]
        assert name.endswith("attn.qkv.b") and cfg.d <= element < 2 * cfg.d, d
    a, b = rg.run(gpu, state, steps=20), rg.run(cpu, state, steps=20)
    close(np.array(a.history["aux"]), np.array(b.history["aux"]), 1e-4, "loss curve")
    # Uniform random tokens carry no structure: the loss stays near ln(vocab).
    assert abs(np.mean(a.history["aux"]) - np.log(cfg.vocab)) < 0.1


def test_small_independent_groups_run_as_one_launch():
    """AdamW over a small MLP: one update group per parameter shape, each far too small to fill
    the device. The runtime launches runs of such independent groups as one kernel; the training
    run must equal the oracle's, and the launch count per pass must drop."""
    import json
    step, state = workloads.mlp_train_step(workloads.MLPConfig(batch=64, d_in=16, hidden=32))
    hip = rg.compile(step, (state,), device="hip", validate="none")
    cpu = rg.compile(step, (state,), device="cpu", validate="none")
    bd = hip.profile(state, repeats=1)["breakdown"]
    per = (json.loads(bd) if isinstance(bd, str) else bd)["per_step"]
    assert per["merged_launches"] >= 1 and per["launches"] < per["dispatches"], per
    a = rg.run(hip, state, steps=20)
    b = rg.run(cpu, state, steps=20)
    close(np.array(a.history["aux"]), np.array(b.history["aux"]), 1e-4, "loss curve")
    from rustautograd_amd import tree as rtree
    for (name, u), (_, v) in zip(rtree.paths(a.state["params"]), rtree.paths(b.state["params"])):
        close(u.numpy(), v.numpy(), 1e-4, name)


def test_device_training_resumes_bit_identically_from_a_checkpoint(tmp_path):
    """The device loop is deterministic: a run checkpointed after 4 steps and resumed for 3 equals
    an uninterrupted 7-step run bit for bit, state and losses (checkpoint format: safetensors,
    reference python/rg/checkpoint.py)."""
    cfg = workloads.GPT_CONFIGS["C3"]._replace(batch=4, block=32, layers=2)
    step, state = workloads.gpt_train_step(cfg)
    c = rg.compile(step, (state,), validate="none", device="hip")
    first = rg.run(c, state, steps=4)
    path = str(tmp_path / "resume.safetensors")
    rg.save(path, first.state)
    resumed = rg.run(c, rg.load(path), steps=3)
    straight = rg.run(c, state, steps=7)
    assert resumed.history["aux"] == straight.history["aux"][4:]
    for (name, u), (_, v) in zip(rg.tree.paths(resumed.state), rg.tree.paths(straight.state)):
        assert u.numpy().tobytes() == v.numpy().tobytes(), name


def test_sampler_on_the_device_matches_the_oracle_token_for_token():
    """The generation loop (examples/gpt.py:50-93 of the reference) on the device: train a small
    GPT on windows of a repeating text, then generate greedily and with a nucleus filter; the
    device's losses overlay the oracle's and its tokens equal the oracle's. Then a random-init
    sampler with block 32 and vocab 96 at temperature 0.8 with top-k and top-p filters draws 40
    tokens, identical on both (the random bits are exact; logits differ by rounding only)."""
    from rustautograd_amd import optim
    text = "abcd" * 100
    chars = sorted(set(text))
    tokens = rg.tensor(np.array([chars.index(ch) for ch in text], dtype=np.int32))
    model = workloads.GPT(vocab=4, block=4, d=16, heads=2, layers=1)
    params = model.init(random.key(0))
    opt = optim.adamw(5e-3, weight_decay=0.0)
    state = {"params": params, "opt": opt.init(params), "key": random.key(1)}
    step = workloads.window_train_step(model, opt, 8)
    runs = {dev: rg.run(rg.compile(step, (state, tokens), device=dev), state, tokens, steps=200) for dev in ("hip", "cpu")}
    close(np.array(runs["hip"].history["aux"]), np.array(runs["cpu"].history["aux"]), 1e-4, "pattern loss curve")
    for kw in ({"top_k": 1}, {"top_p": 0.5}):
        got = {dev: workloads.generate(workloads.compile_sampler(model, runs[dev].state["params"], device=dev, **kw), 4, [0, 1, 2, 3], 8)
               for dev in ("hip", "cpu")}
        assert got["hip"] == got["cpu"], kw
        assert "".join(chars[t] for t in got["hip"]) == "abcdabcd", kw
    big = workloads.GPT(vocab=96, block=32, d=64, heads=2, layers=2)
    big_params = big.init(random.key(3))
    drawn = {dev: workloads.generate(workloads.compile_sampler(big, big_params, temperature=0.8, top_k=20, top_p=0.9, device=dev), 32,
                                     [5, 17, 42], 40, seed=9) for dev in ("hip", "cpu")}
    assert drawn["hip"] == drawn["cpu"]
    assert len(set(drawn["hip"])) > 5
