"""Control flow on the HIP backend: scan, while_loop and cond against the CPU oracle.

A body runs as a program of its own on the execution stream (csrc/hip/runtime.cpp run_scan,
run_while, run_cond): a scan's steps are launches and copies only, so it is captured with the
rest of a step in the run loop's HIP graphs; while and cond read one scalar per decision. The
programs are those of tests/test_control_flow.py (the reference's tests/engine.rs:1108-1310,
tests/test_framework.py:544-697 and tests/metal.rs:395-421). float64 results agree with the
oracle to 1e-12 (device transcendentals are within 2 ulp); float32 to 1e-5 relative.
"""

import json

import numpy as np
import pytest

import rustautograd_amd as rg

from helpers import G
from test_control_flow import (RNN_INPUTS, _cond_graph, _counting_while, _rnn, f64, rnn_loss_loop, rnn_loss_scan)

pytestmark = pytest.mark.gpu


def _both(g, outs, inputs, optimize="standard"):
    return g.eval(outs, inputs, device="hip", optimize=optimize), g.eval(outs, inputs, device="cpu", optimize=optimize)


def test_scan_values_and_gradients_equal_the_oracle_and_the_unrolled_loop():
    g1, o1 = _rnn(True)
    g2, o2 = _rnn(False)
    hip, cpu = _both(g1, o1, RNN_INPUTS)
    unrolled = g2.eval(o2, RNN_INPUTS, device="cpu")
    for k, (a, b, c) in enumerate(zip(hip, cpu, unrolled)):
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-12, err_msg=f"output {k} vs oracle")
        np.testing.assert_allclose(a, c, rtol=0, atol=1e-12, err_msg=f"output {k} vs unrolled")


def test_second_order_gradient_and_integer_carries_through_scan():
    b = G()
    c = b.input((), "float64")
    g = G()
    x = g.input((), "float64")
    node = g.g.scan(b.g, [b.bin("mul", c, c)], 1, 0, 3, [x])
    y = g.g.output(node, 0, [], "float64")
    (d1,) = g.grad(y, [x])
    (d2,) = g.grad(d1, [x])
    r = g.eval([y, d1, d2], [1.5], device="hip")
    assert abs(float(r[0]) - 1.5 ** 8) < 1e-9 and abs(float(r[1]) - 8 * 1.5 ** 7) < 1e-9 and abs(float(r[2]) - 56 * 1.5 ** 6) < 1e-8

    b = G()
    i, xx = b.input((), "int32"), b.input((), "float64")
    g = G()
    i0, x0 = g.const(0, (), "int32"), g.input((), "float64")
    node = g.g.scan(b.g, [b.bin("add", i, b.const(1, (), "int32")), b.bin("mul", xx, b.scalar(2.0))], 2, 0, 4, [i0, x0])
    count, yy = g.g.output(node, 0, [], "int32"), g.g.output(node, 1, [], "float64")
    (gx,) = g.grad(yy, [x0])
    r = g.eval([count, yy, gx], [3.0], device="hip")
    assert int(r[0]) == 4 and float(r[1]) == 48.0 and float(r[2]) == 16.0


def test_while_loop_counts_and_reports_its_limit():
    g, total, count, _ = _counting_while(10.0, 1000)
    r = g.eval([total, count], [0.0, 0.0], device="hip")
    assert float(r[0]) == 45.0 and int(r[1]) == 10
    g, total, count, _ = _counting_while(1e9, 7)
    assert int(g.eval([count], [0.0, 0.0], device="hip")[0]) == 7
    bad = json.loads(g.compile([total], [0.0, 0.0], device="hip", optimize="standard", level="standard").report_json)
    assert bad["status"] == "validation_failed" and bad["diagnostics"][0]["code"] == "WHILE_LIMIT_REACHED"


def test_cond_runs_the_taken_branch_and_finds_diagnostics_inside_it():
    g, y, gx = _cond_graph()
    r = g.eval([y, gx], [1.0, 2.0], device="hip")
    assert abs(float(r[0]) - np.log(2.0)) < 1e-12 and abs(float(r[1]) - 0.5) < 1e-12
    r = g.eval([y, gx], [0.0, 2.0], device="hip")
    assert float(r[0]) == 4.0 and float(r[1]) == 4.0
    c = g.compile([y], [0.0, -1.0], device="hip", optimize="standard", level="standard")
    assert json.loads(c.report_json)["status"] == "ok", c.report_json
    bad = json.loads(c.check([rg.tensor(np.float64(1.0))._t, rg.tensor(np.float64(-1.0))._t]))
    assert bad["diagnostics"][0]["node"]["operation"] == "log"
    assert bad["diagnostics"][0]["node"]["control_flow"]["iteration"] == 0


def test_diagnostics_name_the_iteration_inside_a_scan():
    b = G()
    c = b.input((), "float32")
    e = b.un("exp", c)
    nxt = b.bin("mul", c, b.scalar(2.0, "float32"))
    g = G()
    x = g.input((), "float32")
    node = g.g.scan(b.g, [nxt, e], 1, 0, 12, [x])
    ys = g.g.output(node, 1, [12], "float32")
    rep = json.loads(g.compile([ys], [np.float32(1.0)], device="hip", optimize="standard", level="standard").report_json)
    d = rep["diagnostics"][0]
    assert d["code"] == "NUMERIC_OVERFLOW" and d["node"]["operation"] == "exp" and d["node"]["control_flow"]["iteration"] == 7


def test_reverse_scan_with_stacked_carries_matches_the_oracle():
    b = G()
    c, x = b.input((2,), "float64"), b.input((2,), "float64")
    nxt = b.bin("add", b.bin("mul", c, b.scalar(0.5)), x)
    g = G()
    c0, xs = g.input((2,), "float64"), g.input((4, 2), "float64")
    node = g.g.scan(b.g, [nxt, nxt], 1, 1, 4, [c0, xs], True)
    outs = [g.g.output(node, 0, [2], "float64"), g.g.output(node, 1, [4, 2], "float64"), g.g.output(node, 2, [4, 2], "float64")]
    hip, cpu = _both(g, outs, [np.array([1.0, -1.0]), np.arange(8.0).reshape(4, 2)])
    for a, b2 in zip(hip, cpu):
        np.testing.assert_array_equal(a, b2)


def test_python_rnn_scan_and_gradients_float32():
    """The reference's tests/test_framework.py:689-697 (`test_control_flow_runs_on_metal`): a
    float32 scan RNN and its gradients on the device against the CPU."""
    p = {"w": rg.tensor([0.5, 0.2]), "b": rg.tensor([0.1, -0.1])}
    xs = rg.tensor(np.random.default_rng(0).normal(size=(50, 2)).astype("float32"))
    fn = rg.value_and_grad(rnn_loss_scan)
    cpu, gpu = rg.compile(fn, (p, xs), device="cpu"), rg.compile(fn, (p, xs), device="hip")
    assert gpu.report["status"] == "ok", gpu.report
    (va, ga), (vb, gb) = cpu(p, xs), gpu(p, xs)
    assert float(va) == pytest.approx(float(vb), rel=1e-5)
    for k in ("w", "b"):
        np.testing.assert_allclose(gb[k].numpy(), ga[k].numpy(), rtol=1e-5, atol=1e-6)
    # The unrolled loop on the device gives the same numbers.
    (vc, gc) = rg.compile(rg.value_and_grad(rnn_loss_loop), (p, xs), device="hip", validate="none")(p, xs)
    assert float(vc) == pytest.approx(float(vb), rel=1e-5)


def test_scan_over_matrix_products_and_row_groups():
    """A body with device kernels of every kind: a product, a bias, a layer-norm-like row group
    and a tanh, 16 steps over (64, 128) carries; the gradients run the reverse scan."""
    r = np.random.default_rng(4)
    w = rg.tensor((r.normal(size=(128, 128)) / 12).astype(np.float32))
    bias = rg.tensor(r.normal(size=(128,)).astype(np.float32) * 0.1)
    h0 = rg.tensor(r.normal(size=(64, 128)).astype(np.float32))
    xs = rg.tensor(r.normal(size=(16, 64, 128)).astype(np.float32))

    def loss(w, bias, h0, xs):
        def cell(h, x):
            z = h @ w + bias + x
            z = z - z.mean(axis=-1, keepdims=True)
            z = z / rg.sqrt((z * z).mean(axis=-1, keepdims=True) + 1e-5)
            h = rg.tanh(z)
            return h, (h * h).mean()

        h, ys = rg.scan(cell, h0, xs)
        return h.sum() + ys.sum()

    fn = rg.value_and_grad(loss, argnums=(0, 1, 2))
    cpu = rg.compile(fn, (w, bias, h0, xs), device="cpu", validate="none")
    gpu = rg.compile(fn, (w, bias, h0, xs), device="hip", validate="none")
    (va, ga), (vb, gb) = cpu(w, bias, h0, xs), gpu(w, bias, h0, xs)
    assert float(vb) == pytest.approx(float(va), rel=1e-5)
    for k in range(3):
        a, b = ga[k].numpy(), gb[k].numpy()
        assert np.abs(b - a).max() <= 1e-4 * max(1.0, np.abs(a).max()), f"gradient {k}"


@pytest.mark.parametrize("loop", ["scan", "while"])
def test_control_flow_inside_the_device_step_loop(loop):
    """`run` over a step holding a scan (captured in the run loop's HIP graphs) or a while loop
    (launched directly: it waits for its condition), against the oracle's loop."""
    def step(state):
        if loop == "scan":
            def cell(h, _):
                return rg.tanh(h * state["w"] + 0.1), h.sum()

            h, ys = rg.scan(cell, state["h"], length=6)
            extra = ys.sum()
        else:
            def body(s):
                return {"h": rg.tanh(s["h"] * state["w"] + 0.1), "n": s["n"] + 1.0}

            out = rg.while_loop(lambda s: s["n"] < 6.0, body, {"h": state["h"], "n": f64(0.0)})
            h, extra = out["h"], out["n"]
        loss = (h * h).sum() + extra
        return {"h": h, "w": state["w"] * 0.99}, loss

    state = {"h": f64([0.2, -0.1, 0.4]), "w": f64([0.9, 1.1, 0.7])}
    gpu, cpu = rg.compile(step, (state,), device="hip"), rg.compile(step, (state,), device="cpu")
    a, b = rg.run(gpu, state, steps=7), rg.run(cpu, state, steps=7)
    np.testing.assert_allclose(a.state["h"].numpy(), b.state["h"].numpy(), rtol=1e-12)
    np.testing.assert_allclose(np.array(a.history["aux"]), np.array(b.history["aux"]), rtol=1e-12)
    # Twice more through the cached loop, resuming from the returned state.
    a2, b2 = rg.run(gpu, a.state, steps=3), rg.run(cpu, b.state, steps=3)
    np.testing.assert_allclose(a2.state["h"].numpy(), b2.state["h"].numpy(), rtol=1e-12)
