"""The Python surface as a drop-in for the reference's `rg` package (python/rg/*), on the CPU
oracle: tracing, transformations, the run loop's contract, diagnostics that point at user
source, tensors and indexing, random numbers, layers, optimizers and sampling filters. The
behaviours checked are the ones the reference's tests/test_api.py and tests/test_framework.py
pin; inputs and assertions here are this suite's own.
"""

import json

import numpy as np
import pytest
import torch

import rustautograd_amd as rg
from rustautograd_amd import nn, optim, random


def f64(x):
    return rg.tensor(np.asarray(x, dtype=np.float64))


def _line_of(source):
    path, line = source.rsplit(":", 1)
    return open(path).read().splitlines()[int(line) - 1]


# ---- compile and run ----

def test_regression_trains_to_the_true_weights_and_reports_itself():
    rng = np.random.default_rng(11)
    x = rng.normal(size=(128, 5)).astype(np.float32)
    w_true = rng.normal(size=5).astype(np.float32)
    y = x @ w_true

    def step(w, batch):
        xb, yb = batch
        loss, g = rg.value_and_grad(lambda w: ((xb @ w - yb) ** 2).mean())(w)
        return w - 0.05 * g, loss

    w0 = np.zeros(5, np.float32)
    c = rg.compile(step, (w0, (x, y)), validate="standard")
    assert c.report["status"] == "ok", c.report
    assert json.loads(str(c.report))["status"] == "ok"
    r = rg.run(c, state=w0, data=(x, y), steps=600)
    assert (r.status, r.steps) == ("completed", 600)
    np.testing.assert_allclose(r.state.numpy(), w_true, atol=1e-3)
    assert r.history["aux"][-1] < 1e-4 * r.history["aux"][0]
    info = rg.inspect(r)
    assert info["status"] == "completed" and info["gradients"][0]["norm"] < 1e-2
    json.dumps(info)
    # A batch of another shape is refused, never recompiled behind the user's back.
    with pytest.raises(rg.DiagnosticError) as e:
        rg.run(c, state=w0, data=(x[:16], y[:16]), steps=1)
    assert e.value.diagnostic["code"] == "INPUT_SIGNATURE_MISMATCH"
    assert e.value.diagnostic["observation"]["recompile_required"] is True


def test_state_only_steps_cycle_through_a_list_of_batches():
    w0 = f64([1.0])
    batches = [f64([10.0]), f64([20.0]), f64([30.0])]
    c = rg.compile(lambda w, b: w * 2.0 + b, (w0, batches[0]))
    # 1 -> 12 -> 44 -> 118 -> 246 (the fourth step reuses the first batch)
    assert rg.run(c, state=w0, data=batches, steps=4).state.tolist() == [246.0]
    assert rg.run(c, state=w0, data=batches[1], steps=2).state.tolist() == [64.0]


def test_history_records_scalar_aux_by_path_and_keeps_the_last_aux():
    def step(w):
        return w * 0.5, {"total": w.sum(), "doubled": w * 2.0, "pair": (w[0], w[1])}

    w0 = rg.tensor([2.0, 6.0])
    r = rg.run(rg.compile(step, (w0,)), state=w0, steps=3)
    assert r.history == {"aux.pair.0": [2.0, 1.0, 0.5], "aux.pair.1": [6.0, 3.0, 1.5], "aux.total": [8.0, 4.0, 2.0]}
    assert r.aux["doubled"].tolist() == [1.0, 3.0]


def test_compile_leaves_inputs_alone_and_runs_are_bit_identical():
    rng = np.random.default_rng(3)
    x, y = rng.normal(size=(16, 4)).astype(np.float32), rng.normal(size=16).astype(np.float32)
    w = np.full(4, 0.5, np.float32)
    kept = w.copy()

    def step(w, b):
        v, g = rg.value_and_grad(lambda w: ((b[0] @ w - b[1]) ** 2).mean())(w)
        return w - 0.02 * g, v

    c = rg.compile(step, (w, (x, y)), validate="thorough")
    a, b = rg.run(c, w, (x, y), steps=40), rg.run(c, w, (x, y), steps=40)
    assert np.array_equal(w, kept)
    assert a.state.numpy().tobytes() == b.state.numpy().tobytes() and a.history == b.history


def test_iterator_data_callbacks_and_early_stop():
    def step(w, b):
        return w + b, w.sum()

    w0 = f64([0.0])
    c = rg.compile(step, (w0, f64([1.0])))
    seen = []
    r = rg.run(c, w0, iter([f64([1.0])] * 10), steps=100, every=3, callback=lambda res: seen.append(res.steps))
    assert r.status == "completed" and r.steps == 10 and seen == [3, 6, 9, 10]
    r = rg.run(c, w0, [f64([1.0])], steps=100, every=4, callback=lambda res: res.steps < 8)
    assert r.status == "stopped_by_callback" and r.steps == 8 and r.state.tolist() == [8.0]


def test_a_diverging_run_stops_and_inspect_finds_the_node_and_inputs():
    x = rg.tensor(np.linspace(0.5, 2.0, 16, dtype=np.float32).reshape(-1, 1))
    y = rg.tensor(np.linspace(0.5, 2.0, 16, dtype=np.float32))

    def loss(w, b):
        return ((b[0] @ w - b[1]) ** 2).mean()  # DIVERGES-HERE

    def step(w, b):
        v, g = rg.value_and_grad(loss)(w, b)
        return w - 8.0 * g, v

    w0 = rg.tensor([1.5])
    c = rg.compile(step, (w0, (x, y)))
    r = rg.run(c, w0, (x, y), steps=50_000)
    assert r.status == "stopped_nonfinite" and r.steps < 50_000
    info = rg.inspect(r)
    assert info["status"] == "nonfinite_detected"
    root = next(d for d in info["diagnostics"] if d["severity"] == "error")
    assert root["code"] == "NUMERIC_OVERFLOW"
    src = root["node"]["source"]
    lines = open(src.rsplit(":", 1)[0]).read().splitlines()
    at = int(src.rsplit(":", 1)[1]) - 1
    assert "DIVERGES-HERE" in lines[at] or "DIVERGES-HERE" in lines[at - 1]
    assert info["repro"]["step"] <= r.nonfinite_step
    again = c.check(info.repro_inputs["state"], info.repro_inputs["data"])
    assert again["status"] == "validation_failed" and again["diagnostics"][0]["code"] == root["code"]


# ---- diagnostics point at the user's line ----

def test_shape_errors_name_the_line_that_caused_them():
    def bad(v):
        return v + rg.tensor([1.0, 2.0, 3.0, 4.0])  # SHAPE-LINE

    with pytest.raises(rg.DiagnosticError) as e:
        rg.compile(bad, (rg.tensor([1.0, 2.0]),))
    d = e.value.diagnostic
    assert d["code"] == "SHAPE_MISMATCH" and d["observation"]["lhs_shape"] == [2] and d["observation"]["rhs_shape"] == [4]
    assert d["node"]["source"].rsplit(":", 1)[0] == __file__
    assert "SHAPE-LINE" in _line_of(d["node"]["source"])


def test_python_branches_on_traced_values_are_refused_with_the_remedy():
    with pytest.raises(rg.DiagnosticError) as e:
        rg.compile(lambda v: v * 2.0 if v.max() > 1.0 else v, (rg.tensor([1.0]),))
    assert e.value.diagnostic["code"] == "CONTROL_FLOW_ON_TRACER"
    assert "rg_where" in e.value.diagnostic["diagnosis"]["cause"]


def test_leaked_tracers_and_mixed_dtypes_are_errors():
    kept = []
    rg.compile(lambda v: kept.append(v) or v, (rg.tensor([1.0]),))
    with pytest.raises(rg.DiagnosticError) as e:
        kept[0] * 2.0
    assert e.value.diagnostic["code"] == "TRACER_LEAK"
    with pytest.raises(rg.DiagnosticError) as e:
        rg.tensor([1.0]) + rg.tensor([1.0], "float64")
    assert e.value.diagnostic["code"] == "DTYPE_MISMATCH"
    with pytest.raises(rg.DiagnosticError) as e:
        rg.arange(3) * 0.5
    assert e.value.diagnostic["code"] == "DTYPE_MISMATCH"


def test_a_failed_validation_blocks_the_run_and_names_the_source():
    c = rg.compile(lambda v: v.exp(), (rg.tensor([95.0]),))  # OVERFLOW-LINE
    assert c.report["status"] == "validation_failed"
    d = c.report["diagnostics"][0]
    assert d["code"] == "NUMERIC_OVERFLOW" and d["observation"]["input_max"] == 95.0
    assert d["diagnosis"] == {"cause": "exponential_overflow", "certainty": "verified"}
    assert "OVERFLOW-LINE" in _line_of(d["node"]["source"])
    with pytest.raises(rg.DiagnosticError):
        rg.run(c, state=rg.tensor([1.0]), steps=1)


def test_a_backward_trap_is_reported_at_its_forward_source():
    def f(v):
        return rg.where(v > 0.0, rg.log(v), 0.0).sum()  # TRAP-LINE

    c = rg.compile(rg.grad(f), (f64([0.0, 2.0]),))
    d = next(x for x in c.report["diagnostics"] if x["severity"] == "error")
    assert d["node"]["role"] == "backward" and d["node"]["forward_node"]["operation"] == "log"
    assert "TRAP-LINE" in _line_of(d["node"]["source"])


def test_unknown_devices_are_refused():
    assert "cpu" in rg.devices()
    with pytest.raises(rg.DiagnosticError) as e:
        rg.compile(lambda v: v, (rg.tensor([1.0]),), device="quantum")
    assert e.value.diagnostic["code"] == "DEVICE_UNAVAILABLE"


def test_the_memory_warning_fires_when_the_plan_fills_the_device(monkeypatch):
    from rustautograd_amd import _native, program
    monkeypatch.setattr(_native, "device_memory_bytes", lambda device: 1 << 30)
    monkeypatch.setattr(program, "MEMORY_WARNING_FRACTION", 0.0)
    c = rg.compile(lambda a: (a @ a).tanh().sum(), (rg.zeros((64, 64)),), validate="none")
    d = next(d for d in c.report["diagnostics"] if d["code"] == "PLAN_NEAR_PHYSICAL_MEMORY")
    assert d["severity"] == "warning" and c.report["status"] == "warning" and c.report.ok


# ---- transformations ----

def test_gradients_of_trees_match_torch():
    rng = np.random.default_rng(4)
    p = {"a": rng.normal(size=(3, 5)), "b": rng.normal(size=5), "c": [rng.normal(size=(5, 2))]}
    x = rng.normal(size=(7, 3))

    def loss(p):
        h = rg.tanh(rg.tensor(x) @ p["a"] + p["b"]) if not torch.is_tensor(p["a"]) else torch.tanh(torch.tensor(x) @ p["a"] + p["b"])
        return ((h @ p["c"][0]) ** 2).mean()

    value, g = rg.value_and_grad(loss)(p)
    tp = {"a": torch.tensor(p["a"], requires_grad=True), "b": torch.tensor(p["b"], requires_grad=True),
          "c": [torch.tensor(p["c"][0], requires_grad=True)]}
    tv = loss(tp)
    tv.backward()
    assert float(value) == pytest.approx(tv.item(), rel=1e-12)
    np.testing.assert_allclose(g["a"].numpy(), tp["a"].grad.numpy(), rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(g["b"].numpy(), tp["b"].grad.numpy(), rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(g["c"][0].numpy(), tp["c"][0].grad.numpy(), rtol=1e-11, atol=1e-13)


def test_higher_order_jvp_hessian_and_custom_rules():
    third = rg.grad(rg.grad(rg.grad(lambda v: v ** 5)))
    assert float(third(f64(1.0))) == 60.0
    y, t = rg.jvp(lambda v: (v * v).sum(), (f64([3.0, 4.0]),), (f64([0.0, 1.0]),))
    assert float(y) == 25.0 and float(t) == 8.0
    np.testing.assert_allclose(rg.hessian(lambda v: (v * v * v).sum())(f64([2.0, -1.0])).numpy(), [[12.0, 0.0], [0.0, -6.0]])
    halve = rg.custom_vjp(lambda v: v, lambda args, out, ct: (ct * 0.5,))
    assert rg.grad(lambda v: (halve(v) * 4.0).sum())(f64([1.0, 1.0])).tolist() == [2.0, 2.0]
    g, aux = rg.grad(lambda v: ((v * v).sum(), v + 1.0), has_aux=True)(f64([2.0]))
    assert g.tolist() == [4.0] and aux.tolist() == [3.0]
    ga, gb = rg.grad(lambda a, b: (a * b * b).sum(), argnums=(0, 1))(f64([2.0]), f64([3.0]))
    assert ga.tolist() == [9.0] and gb.tolist() == [12.0]
    wrong = rg.custom_vjp(lambda v: v, lambda args, out, ct: (ct.sum(),))
    with pytest.raises(rg.DiagnosticError) as e:
        rg.grad(lambda v: wrong(v).sum())(f64([1.0, 2.0]))
    assert e.value.diagnostic["code"] == "CUSTOM_VJP_MISMATCH"


def test_disconnected_and_flat_gradients_are_reported():
    cut = rg.compile(rg.grad(lambda p: p[1].sum()), ((rg.tensor([1.0]), rg.tensor([2.0])),))
    assert any(d["code"] == "GRAD_DISCONNECTED" for d in cut.report["diagnostics"])
    flat = rg.compile(rg.grad(lambda v: rg.minimum(v, -3.0).sum()), (rg.tensor([1.0, 2.0]),))
    d = next(d for d in flat.report["diagnostics"] if d["code"] == "GRAD_ALL_ZERO")
    assert d["diagnosis"]["certainty"] == "suspected"


# ---- tensors, indexing, integers ----

def test_tensor_construction_and_conversion():
    a = np.arange(12, dtype=np.float64).reshape(3, 4)
    t = rg.tensor(a)
    assert t.dtype == "float64" and np.array_equal(np.asarray(t), a)
    assert rg.tensor(np.arange(4, dtype=np.int64)).dtype == "int32"
    assert rg.tensor([True, False]).dtype == "int32"
    assert rg.tensor(2.5).shape == () and rg.tensor(7).dtype == "int32" and rg.tensor([1, 2.5]).dtype == "float32"
    with pytest.raises(rg.DiagnosticError) as e:
        rg.tensor([[1.0], [2.0, 3.0]])
    assert e.value.diagnostic["diagnosis"]["cause"] == "ragged_nested_sequence"
    assert float(rg.tensor([[1.0, 2.0], [3.0, 4.0]]).mean()) == 2.5
    assert (rg.tensor([[1.0, 2.0], [3.0, 4.0]]).T[1] + 1).tolist() == [3.0, 5.0]


def test_indexing_forms():
    x = rg.tensor(np.arange(24, dtype=np.float32).reshape(2, 3, 4))
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    for key in [1, -1, (0, 2), (slice(None), 1), (Ellipsis, 3), (None, 1), (1, None, slice(1, 3)), (slice(None, None, 2),),
                (0, slice(None, None, -1)), (slice(None), slice(0, 3, 2), Ellipsis), (Ellipsis, None)]:
        np.testing.assert_array_equal(x[key].numpy(), a[key], err_msg=repr(key))
    np.testing.assert_array_equal(x[rg.tensor([1, 0, 1])].numpy(), a[[1, 0, 1]])
    np.testing.assert_array_equal(x[[0]].numpy(), a[[0]])
    with pytest.raises(rg.DiagnosticError) as e:
        x[2]
    assert e.value.diagnostic["code"] == "INVALID_SLICE"
    with pytest.raises(rg.DiagnosticError):
        x[0, 0, 0, 0]


def test_integer_tensors_selection_and_shapes():
    assert (rg.arange(4) * rg.arange(4) - 1).tolist() == [-1, 0, 3, 8]
    x = rg.tensor([[4.0, 1.0], [2.0, 8.0], [6.0, 3.0]])
    assert rg.take(x, rg.tensor([0]), axis=1).tolist() == [[4.0], [2.0], [6.0]]
    assert rg.take_along_axis(x, rg.tensor([[1], [1], [0]])).tolist() == [[1.0], [8.0], [6.0]]
    assert rg.argmax(x).tolist() == [0, 1, 0] and rg.argmax(x, axis=0).tolist() == [2, 1] and int(rg.argmax(x, axis=None)) == 3
    assert rg.equal(rg.arange(3), rg.tensor([0, 2, 2])).tolist() == [1, 0, 1]
    assert rg.not_equal(rg.arange(3), rg.tensor([0, 2, 2])).tolist() == [0, 1, 0]
    assert rg.stack([x, x], axis=1).shape == (3, 2, 2) and rg.concatenate([x, x]).shape == (6, 2)
    assert rg.squeeze(x[:, None, :]).shape == (3, 2) and rg.expand_dims(x, -1).shape == (3, 2, 1)
    assert rg.flip(rg.arange(4)).tolist() == [3, 2, 1, 0]
    assert rg.clip(x, 2.0, 5.0).tolist() == [[4.0, 2.0], [2.0, 5.0], [5.0, 3.0]]
    with pytest.raises(rg.DiagnosticError) as e:
        rg.arange(3).exp()
    assert e.value.diagnostic["code"] == "UNSUPPORTED_DTYPE"


def test_sorting_matches_numpy_and_torch_with_gradients():
    rng = np.random.default_rng(9)
    a = rng.normal(size=(3, 7))
    x = f64(a)
    np.testing.assert_array_equal(rg.sort(x).numpy(), np.sort(a, -1))
    np.testing.assert_array_equal(rg.sort(x, axis=0, descending=True).numpy(), -np.sort(-a, 0))
    np.testing.assert_array_equal(rg.argsort(x).numpy(), np.argsort(a, -1, kind="stable"))
    values, idx = rg.top_k(x, 4)
    tv, ti = torch.topk(torch.tensor(a), 4)
    np.testing.assert_array_equal(values.numpy(), tv.numpy())
    np.testing.assert_array_equal(idx.numpy(), ti.numpy())
    np.testing.assert_allclose(rg.cumsum(x, axis=0).numpy(), np.cumsum(a, 0))
    assert rg.argsort(rg.tensor([3.0, float("nan"), -1.0])).tolist() == [2, 0, 1]
    ta = torch.tensor(a, requires_grad=True)
    (torch.sort(ta, -1)[0] * torch.arange(7.0, dtype=torch.float64)).sum().backward()
    g = rg.grad(lambda v: (rg.sort(v) * f64(np.arange(7.0))).sum())(x)
    np.testing.assert_allclose(g.numpy(), ta.grad.numpy())


# ---- random ----

def test_random_draws_are_pure_functions_of_their_key():
    k = random.key(123)
    assert random.normal(k, (5,)).tolist() == random.normal(k, (5,)).tolist()
    k1, k2 = random.split(k)
    assert k1.tolist() != k2.tolist() and random.split(k, 4).shape == (4, 2)
    ints = random.randint(k, (30000,), -2, 3).numpy()
    assert ints.dtype == np.int32 and ints.min() == -2 and ints.max() == 2
    assert np.abs(np.bincount(ints + 2) / 30000 - 0.2).max() < 0.015
    probs = np.array([0.1, 0.6, 0.3])
    draws = random.categorical(k, rg.tensor(np.log(probs)[None, :] * np.ones((40000, 1)), "float32")).numpy()
    np.testing.assert_allclose(np.bincount(draws) / 40000, probs, atol=0.015)
    assert abs(random.bernoulli(k, 0.7, (20000,)).numpy().mean() - 0.7) < 0.015
    u = random.uniform(k, (2000,), low=-1.0, high=1.0).numpy()
    assert -1.0 <= u.min() and u.max() < 1.0
    g = random.gumbel(k, (20000,), "float64").numpy()
    assert abs(g.mean() - 0.5772156649) < 0.03
    with pytest.raises(rg.DiagnosticError) as e:
        random.uniform(rg.tensor([1, 2, 3]), (2,))
    assert e.value.diagnostic["code"] == "INVALID_KEY"


def test_a_key_carried_in_the_state_advances_and_replays():
    def step(s):
        k_next, k_draw = random.split(s["key"])
        return {"key": k_next, "acc": s["acc"] + random.uniform(k_draw, (2,))}, s["acc"].sum()

    s0 = {"key": random.key(5), "acc": rg.zeros(2)}
    c = rg.compile(step, (s0,))
    a, b = rg.run(c, s0, steps=15), rg.run(c, s0, steps=15, every=4, callback=lambda r: None)
    assert a.state["acc"].tolist() == b.state["acc"].tolist() and a.history == b.history
    assert len(set(a.history["aux"])) == 15


# ---- layers, losses, optimizers ----

def test_layers_compose_and_count_parameters():
    key = random.key(2)
    model = nn.Sequential(nn.Linear(6, 10), nn.silu, nn.Linear(10, 3, bias=False))
    p = model.init(key)
    assert sorted(p) == ["0", "2"] and model(p, rg.zeros((4, 6))).shape == (4, 3)
    assert rg.tree.size(p) == 6 * 10 + 10 + 10 * 3
    assert [name for name, _ in rg.tree.paths(p)] == ["0.b", "0.w", "2.w"]
    assert [name for name, _ in rg.tree.paths(p, "model.")] == ["model.0.b", "model.0.w", "model.2.w"]
    cell = nn.GRUCell(2, 4)
    pc = cell.init(key)
    h = rg.zeros((3, 4))
    for _ in range(4):
        h = cell(pc, rg.ones((3, 2)), h)
    assert h.shape == (3, 4) and np.all(np.abs(h.numpy()) < 1.0)
    g = rg.grad(lambda q: cell(q, rg.ones((3, 2)), rg.ones((3, 4)) * 0.5).sum())(pc)
    assert float(rg.tree.global_norm(g)) > 0.0
    with pytest.raises(ValueError):
        nn.MultiHeadAttention(12, 5)


def test_losses_and_activations_match_torch():
    rng = np.random.default_rng(6)
    z = rng.normal(size=(5, 7)) * 3.0
    labels = rng.integers(0, 7, size=5)
    tz = torch.tensor(z)
    F = torch.nn.functional
    close = lambda a, b: np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-12, atol=1e-14)
    close(nn.softmax(f64(z)), F.softmax(tz, -1))
    close(nn.log_softmax(f64(z), axis=0), F.log_softmax(tz, 0))
    close(nn.logsumexp(f64(z)), torch.logsumexp(tz, -1))
    close(nn.gelu(f64(z)), F.gelu(tz, approximate="tanh"))
    close(nn.silu(f64(z)), F.silu(tz))
    close(nn.softplus(f64(z)), F.softplus(tz))
    close(nn.relu(f64(z)), F.relu(tz))
    assert float(nn.cross_entropy(f64(z), rg.tensor(labels.astype(np.int32)))) == pytest.approx(
        F.cross_entropy(tz, torch.tensor(labels)).item(), rel=1e-12)
    t = (rng.uniform(size=(5, 7)) > 0.5).astype(np.float64)
    assert float(nn.binary_cross_entropy_with_logits(f64(z), f64(t))) == pytest.approx(
        F.binary_cross_entropy_with_logits(tz, torch.tensor(t)).item(), rel=1e-12)
    assert float(nn.accuracy(f64(z), rg.tensor(labels.astype(np.int32)))) == pytest.approx(np.mean(z.argmax(-1) == labels))
    assert nn.one_hot(rg.tensor([2, 0]), 3).tolist() == [[0.0, 0.0, 1.0], [1.0, 0.0, 0.0]]


def test_clipping_and_the_cosine_schedule():
    g = {"u": f64([6.0, 0.0]), "v": f64([8.0])}
    clipped = optim.clip_by_global_norm(g, 5.0)
    assert float(rg.tree.global_norm(clipped)) == pytest.approx(5.0)
    assert clipped["u"].tolist() == pytest.approx([3.0, 0.0])
    assert optim.clip_by_global_norm(g, 50.0)["v"].tolist() == [8.0]
    s = optim.cosine_decay(2.0, 104, warmup_steps=4, min_lr=0.2)
    assert float(s(f64(0.0))) == pytest.approx(0.5)        # warm-up: 2 * 1/4
    assert float(s(f64(3.0))) == pytest.approx(2.0)
    assert float(s(f64(54.0))) == pytest.approx(1.1)       # half-way down the cosine
    assert float(s(f64(104.0))) == pytest.approx(0.2) and float(s(f64(1000.0))) == pytest.approx(0.2)


def test_sgd_momentum_and_rmsprop_follow_torch():
    rng = np.random.default_rng(12)
    p0 = {"w": rng.normal(size=(4, 3)), "b": rng.normal(size=3)}
    x = rng.normal(size=(8, 4))

    def loss(p):
        return ((rg.tensor(x) @ p["w"] + p["b"]) ** 2).mean()

    for make, tmake in ((lambda: optim.sgd(0.05, momentum=0.8), lambda ps: torch.optim.SGD(ps, lr=0.05, momentum=0.8)),
                        (lambda: optim.rmsprop(0.01, decay=0.9, eps=1e-8), lambda ps: torch.optim.RMSprop(ps, lr=0.01, alpha=0.9, eps=1e-8))):
        opt = make()
        p, s = {k: f64(v) for k, v in p0.items()}, None
        s = opt.init(p)
        tp = {k: torch.tensor(v, requires_grad=True) for k, v in p0.items()}
        topt = tmake(list(tp.values()))
        for _ in range(5):
            g = rg.grad(loss)(p)
            p, s = opt.update(g, s, p)
            topt.zero_grad()
            ((torch.tensor(x) @ tp["w"] + tp["b"]) ** 2).mean().backward()
            topt.step()
        for k in p0:
            np.testing.assert_allclose(p[k].numpy(), tp[k].detach().numpy(), rtol=1e-10, atol=1e-12)


def test_sampling_filters_keep_the_right_tokens():
    probs = np.array([[0.4, 0.25, 0.2, 0.1, 0.05]])
    logits = f64(np.log(probs))
    kept = lambda out: (out.numpy() > -1e8).tolist()[0]
    assert kept(nn.top_k_logits(logits, 3)) == [True, True, True, False, False]
    assert kept(nn.top_p_logits(logits, 0.5)) == [True, True, False, False, False]
    assert kept(nn.top_p_logits(logits, 0.4)) == [True, False, False, False, False]
    assert kept(nn.top_p_logits(logits, 0.86)) == [True, True, True, True, False]
    shuffled = f64(np.log([[0.1, 0.05, 0.4, 0.2, 0.25]]))
    assert kept(nn.top_p_logits(shuffled, 0.6)) == [False, False, True, False, True]
    c = rg.compile(lambda k: random.categorical(k, nn.top_k_logits(rg.tensor(np.log([[0.5, 0.2, 0.3]] * 400), "float32"), 2)),
                   (random.key(0),))
    assert set(c(random.key(3)).tolist()) == {0, 2}
