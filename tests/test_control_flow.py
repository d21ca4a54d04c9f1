"""Control flow: scan, while_loop and cond, through the engine and the Python surface.

Mirrors the reference's tests/engine.rs:1108-1310 (graph level) and tests/test_framework.py:
544-697 (Python level). Values are checked against independent computations: the same loop
unrolled into plain nodes, numpy or torch in float64, closed forms (x^(2^3) and its first two
derivatives), and central differences. These run on the CPU oracle with the CPU plan ("cpu") and
with the device-flavoured plan ("cpu_devplan"); tests/test_hip_control_flow.py runs the same
programs on the HIP backend.
"""

import numpy as np
import pytest
import torch

import rustautograd_amd as rg
from rustautograd_amd import random

from conftest import DEVPLAN
from helpers import G

DEVICES = ["cpu", DEVPLAN]


def f64(x):
    return rg.tensor(np.asarray(x, dtype=np.float64), "float64")


# ---- graph level (tests/engine.rs) ---------------------------------------------------------------

def _rnn_body(d):
    b = G()
    c, x, w = b.input((d,), "float64"), b.input((d,), "float64"), b.input((d,), "float64")
    nxt = b.un("tanh", b.bin("add", b.bin("mul", c, w), x))
    return b, [nxt, b.bin("mul", nxt, nxt)]


def _rnn(use_scan, d=3, length=5):
    g = G()
    c0, xs, w = g.input((d,), "float64"), g.input((length, d), "float64"), g.input((d,), "float64")
    if use_scan:
        b, outs = _rnn_body(d)
        node = g.g.scan(b.g, outs, 1, 1, length, [c0, xs, w])
        last = g.g.output(node, 0, [d], "float64")
        ys = g.g.output(node, 1, [length, d], "float64")
    else:
        c, rows = c0, []
        for k in range(length):
            x = g.op("reshape", [g.op("slice", [xs], starts=[k, 0], stops=[k + 1, d])], shape=[d])
            c = g.un("tanh", g.bin("add", g.bin("mul", c, w), x))
            rows.append(g.op("reshape", [g.bin("mul", c, c)], shape=[1, d]))
        last, ys = c, g.op("concat", rows, axis=0)
    y = g.bin("add", g.sum_all(last), g.sum_all(ys))
    return g, [last, ys, y] + g.grad(y, [c0, xs, w])


RNN_INPUTS = [np.array([0.1, -0.2, 0.3]), np.sin(np.arange(15) * 0.7).reshape(5, 3), np.array([0.5, 0.9, -0.4])]


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("optimize", ["none", "standard"])
def test_scan_values_and_gradients_equal_the_unrolled_loop(device, optimize):
    g1, o1 = _rnn(True)
    g2, o2 = _rnn(False)
    a = g1.eval(o1, RNN_INPUTS, device=device, optimize=optimize)
    b = g2.eval(o2, RNN_INPUTS, device="cpu")
    for k, (u, v) in enumerate(zip(a, b)):
        assert u.shape == v.shape
        np.testing.assert_allclose(u, v, rtol=0, atol=1e-12, err_msg=f"output {k}")


def test_scan_gradients_match_torch():
    g, outs = _rnn(True)
    got = g.eval(outs, RNN_INPUTS)
    c0, xs, w = (torch.tensor(x, requires_grad=True) for x in RNN_INPUTS)
    c, ys = c0, []
    for k in range(5):
        c = torch.tanh(c * w + xs[k])
        ys.append(c * c)
    y = c.sum() + torch.stack(ys).sum()
    y.backward()
    for k, t in enumerate((c0, xs, w)):
        np.testing.assert_allclose(got[3 + k], t.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_scan_validates_thoroughly():
    g, outs = _rnn(True)
    c = g.compile(outs, RNN_INPUTS, device="cpu", optimize="standard", level="thorough")
    import json
    report = json.loads(c.report_json)
    assert report["status"] == "ok", report
    grad_check = next(ch for ch in report["checks"] if ch["name"] == "grad_check")
    assert grad_check["detail"]["elements_checked"] > 5


@pytest.mark.parametrize("device", DEVICES)
def test_second_order_gradient_through_scan(device):
    # Repeated squaring: x -> x^(2^3) = x^8, with 8 x^7 and 56 x^6 in closed form.
    b = G()
    c = b.input((), "float64")
    g = G()
    x = g.input((), "float64")
    node = g.g.scan(b.g, [b.bin("mul", c, c)], 1, 0, 3, [x])
    y = g.g.output(node, 0, [], "float64")
    (d1,) = g.grad(y, [x])
    (d2,) = g.grad(d1, [x])
    r = g.eval([y, d1, d2], [1.5], device=device)
    assert abs(float(r[0]) - 1.5 ** 8) < 1e-9
    assert abs(float(r[1]) - 8 * 1.5 ** 7) < 1e-9
    assert abs(float(r[2]) - 56 * 1.5 ** 6) < 1e-8


@pytest.mark.parametrize("device", DEVICES)
def test_integer_carries_flow_through_scan_and_gradients(device):
    b = G()
    i, x = b.input((), "int32"), b.input((), "float64")
    ni = b.bin("add", i, b.const(1, (), "int32"))
    nx = b.bin("mul", x, b.scalar(2.0))
    g = G()
    i0, x0 = g.const(0, (), "int32"), g.input((), "float64")
    node = g.g.scan(b.g, [ni, nx], 2, 0, 4, [i0, x0])
    count = g.g.output(node, 0, [], "int32")
    y = g.g.output(node, 1, [], "float64")
    (gx,) = g.grad(y, [x0])
    r = g.eval([count, y, gx], [3.0], device=device)
    assert int(r[0]) == 4 and float(r[1]) == 48.0 and float(r[2]) == 16.0


def _counting_while(limit, max_iterations):
    cg = G()
    i, _ = cg.input((), "float64"), cg.input((), "float64")
    c = cg.bin("gt", cg.scalar(limit), i)
    bg = G()
    i2, s2 = bg.input((), "float64"), bg.input((), "float64")
    ni = bg.bin("add", i2, bg.scalar(1.0))
    ns = bg.bin("add", s2, i2)
    g = G()
    i0, s0 = g.input((), "float64"), g.input((), "float64")
    node = g.g.while_loop(cg.g, c, bg.g, [ni, ns], 2, max_iterations, [i0, s0])
    total = g.g.output(node, 1, [], "float64")
    count = g.g.output(node, 2, [], "int32")
    return g, total, count, i0


@pytest.mark.parametrize("device", DEVICES)
def test_while_loop_runs_to_its_condition_and_reports_the_limit(device):
    g, total, count, _ = _counting_while(10.0, 1000)
    r = g.eval([total, count], [0.0, 0.0], device=device)
    assert float(r[0]) == 45.0 and int(r[1]) == 10
    import json
    ok = json.loads(g.compile([total], [0.0, 0.0], device=device, optimize="standard", level="standard").report_json)
    assert ok["status"] == "ok", ok

    g, total, count, _ = _counting_while(1e9, 7)
    assert int(g.eval([count], [0.0, 0.0], device=device)[0]) == 7
    bad = json.loads(g.compile([total], [0.0, 0.0], device=device, optimize="standard", level="standard").report_json)
    assert bad["status"] == "validation_failed"
    assert bad["diagnostics"][0]["code"] == "WHILE_LIMIT_REACHED"
    assert bad["diagnostics"][0]["observation"]["max_iterations"] == 7

    g, total, _, x = _counting_while(5.0, 100)
    with pytest.raises(rg.DiagnosticError) as e:
        g.grad(total, [x])
    assert e.value.diagnostic["code"] == "GRAD_THROUGH_WHILE"


def _branch(f):
    b = G()
    x = b.input((), "float64")
    return b, f(b, x)


def _cond_graph():
    tb, to = _branch(lambda b, x: b.un("log", x))
    eb, eo = _branch(lambda b, x: b.bin("mul", x, x))
    g = G()
    p, x = g.input((), "float64"), g.input((), "float64")
    node = g.g.cond(tb.g, [to], eb.g, [eo], [p, x])
    y = g.g.output(node, 0, [], "float64")
    (gx,) = g.grad(y, [x])
    return g, y, gx


@pytest.mark.parametrize("device", DEVICES)
def test_cond_runs_only_the_taken_branch_and_differentiates_it(device):
    import json
    g, y, gx = _cond_graph()
    r = g.eval([y, gx], [1.0, 2.0], device=device)
    assert abs(float(r[0]) - np.log(2.0)) < 1e-12 and abs(float(r[1]) - 0.5) < 1e-12
    r = g.eval([y, gx], [0.0, 2.0], device=device)
    assert float(r[0]) == 4.0 and float(r[1]) == 4.0
    # log(-1) sits in the branch not taken: no NaN, no diagnostic, unlike `where`.
    c = g.compile([y], [0.0, -1.0], device=device, optimize="standard", level="standard")
    assert json.loads(c.report_json)["status"] == "ok", c.report_json
    # Taken, it is found inside the branch.
    bad = json.loads(c.check([rg.tensor(np.float64(1.0))._t, rg.tensor(np.float64(-1.0))._t]))
    assert bad["status"] == "validation_failed"
    assert bad["diagnostics"][0]["node"]["operation"] == "log"
    assert bad["diagnostics"][0]["node"]["control_flow"]["iteration"] == 0


@pytest.mark.parametrize("device", DEVICES)
def test_diagnostics_name_the_iteration_inside_a_scan(device):
    import json
    b = G()
    c = b.input((), "float32")
    e = b.un("exp", c)
    nxt = b.bin("mul", c, b.scalar(2.0, "float32"))
    g = G()
    x = g.input((), "float32")
    node = g.g.scan(b.g, [nxt, e], 1, 0, 12, [x])
    ys = g.g.output(node, 1, [12], "float32")
    rep = json.loads(g.compile([ys], [np.float32(1.0)], device=device, optimize="standard", level="standard").report_json)
    d = rep["diagnostics"][0]
    assert rep["status"] == "validation_failed"
    assert d["code"] == "NUMERIC_OVERFLOW" and d["node"]["operation"] == "exp"
    # 2^7 = 128 is the first value past float32's exp limit of about 88.7.
    assert d["node"]["control_flow"]["iteration"] == 7


@pytest.mark.parametrize("device", DEVICES)
def test_reverse_scan_and_stacked_carries(device):
    """A reverse scan visits positions from the last; the carries before each step come back
    stacked (result index n_carry + n_y), the form second-order gradients read."""
    b = G()
    c, x = b.input((2,), "float64"), b.input((2,), "float64")
    nxt = b.bin("add", b.bin("mul", c, b.scalar(0.5)), x)
    g = G()
    c0, xs = g.input((2,), "float64"), g.input((4, 2), "float64")
    node = g.g.scan(b.g, [nxt, nxt], 1, 1, 4, [c0, xs], True)
    last = g.g.output(node, 0, [2], "float64")
    ys = g.g.output(node, 1, [4, 2], "float64")
    before = g.g.output(node, 2, [4, 2], "float64")
    cv, xv = np.array([1.0, -1.0]), np.arange(8.0).reshape(4, 2)
    r = g.eval([last, ys, before], [cv, xv], device=device)
    want_ys, want_before, cc = np.zeros((4, 2)), np.zeros((4, 2)), cv.copy()
    for at in (3, 2, 1, 0):
        want_before[at] = cc
        cc = cc * 0.5 + xv[at]
        want_ys[at] = cc
    np.testing.assert_array_equal(r[0], cc)
    np.testing.assert_array_equal(r[1], want_ys)
    np.testing.assert_array_equal(r[2], want_before)


# ---- Python surface (tests/test_framework.py) -------------------------------------------------

def rnn_loss_scan(p, xs):
    def cell(h, x):
        h = rg.tanh(h * p["w"] + x + p["b"])
        return h, h * h

    last, ys = rg.scan(cell, rg.zeros_like(p["b"]), xs)
    return last.sum() + ys.mean()


def rnn_loss_loop(p, xs):
    h, total = rg.zeros_like(p["b"]), []
    for k in range(xs.shape[0]):
        h = rg.tanh(h * p["w"] + xs[k] + p["b"])
        total.append(h * h)
    return h.sum() + rg.stack(total).mean()


def test_scan_gradient_equals_the_python_loop_and_torch():
    r = np.random.default_rng(9)
    p = {"w": f64(r.normal(size=3)), "b": f64(r.normal(size=3))}
    xs = f64(r.normal(size=(20, 3)))
    v1, g1 = rg.value_and_grad(rnn_loss_scan)(p, xs)
    v2, g2 = rg.value_and_grad(rnn_loss_loop)(p, xs)
    assert float(v1) == pytest.approx(float(v2), rel=1e-13)
    tp = {k: torch.tensor(v.numpy(), requires_grad=True) for k, v in p.items()}
    txs, h, total = torch.tensor(xs.numpy()), torch.zeros(3, dtype=torch.float64), []
    for k in range(20):
        h = torch.tanh(h * tp["w"] + txs[k] + tp["b"])
        total.append(h * h)
    tv = h.sum() + torch.stack(total).mean()
    tv.backward()
    assert float(v1) == pytest.approx(tv.item(), rel=1e-13)
    for k in p:
        np.testing.assert_allclose(g1[k].numpy(), g2[k].numpy(), rtol=1e-11)
        np.testing.assert_allclose(g1[k].numpy(), tp[k].grad.numpy(), rtol=1e-11)


def test_scan_keeps_the_graph_small_and_validates():
    p = {"w": rg.tensor([0.5, 0.2]), "b": rg.tensor([0.1, -0.1])}
    xs = rg.tensor(np.random.default_rng(0).normal(size=(500, 2)).astype("float32"))
    compact = rg.compile(rg.grad(rnn_loss_scan), (p, xs), validate="thorough")
    unrolled = rg.compile(rg.grad(rnn_loss_loop), (p, xs), validate="none")
    assert compact.report["status"] == "ok", compact.report
    assert compact.report["graph"]["optimization"]["nodes_after"] * 20 < unrolled.report["graph"]["optimization"]["nodes_after"]
    assert next(c for c in compact.report["checks"] if c["name"] == "grad_check")["detail"]["elements_checked"] == 4


def test_scan_structures_captures_and_errors():
    # Trees in carry, x and y; a captured outer value; no xs.
    scale = rg.tensor(2.0, "float64")

    def body(c, x):
        return {"a": c["a"] + x["v"] * scale, "n": c["n"]}, {"out": c["a"]}

    c0 = {"a": f64([0.0]), "n": f64([5.0])}
    final, ys = rg.scan(body, c0, {"v": f64([[1.0], [2.0], [3.0]])})
    assert final["a"].tolist() == [12.0] and final["n"].tolist() == [5.0]
    assert ys["out"].numpy().tolist() == [[0.0], [2.0], [6.0]]
    last, none = rg.scan(lambda c, _: (c * 2.0, None), f64(1.0), length=4)
    assert float(last) == 16.0 and none is None

    for bad in (lambda: rg.scan(lambda c, _: (c.reshape(1, 1), None), f64([1.0]), length=2),
                lambda: rg.scan(lambda c, _: (c, None), f64([1.0])),
                lambda: rg.scan(lambda c, x: (c, x), f64([1.0]), (f64([1.0, 2.0]), f64([1.0])))):
        with pytest.raises(rg.DiagnosticError) as e:
            bad()
        assert e.value.diagnostic["code"] == "CONTROL_FLOW_SHAPE_MISMATCH"
    # An ordinary Python `if` on a traced value is still refused inside a body, with the remedy.
    with pytest.raises(rg.DiagnosticError) as e:
        rg.scan(lambda c, _: (c if c.sum() > 0 else -c, None), f64([1.0]), length=2)
    assert e.value.diagnostic["code"] == "CONTROL_FLOW_ON_TRACER"


def test_nested_scan_in_a_training_step_with_random_keys():
    def inner(c, _):
        return c * 0.5 + 1.0, None

    def outer(c, x):
        k1, k2 = random.split(c["key"])
        h, _ = rg.scan(inner, c["h"] + x + random.normal(k1, (2,), "float64") * 0.0, length=3)
        return {"key": k2, "h": h}, h.sum()

    def loss(w, xs):
        final, ys = rg.scan(outer, {"key": random.key(0), "h": w}, xs)
        return final["h"].sum() + ys.sum()

    w = f64([0.3, 0.4])
    xs = f64(np.ones((4, 2)))
    g = rg.grad(loss)(w, xs)
    h = 1e-6
    for i in range(2):
        d = np.zeros(2)
        d[i] = h
        numeric = (float(loss(f64(w.numpy() + d), xs)) - float(loss(f64(w.numpy() - d), xs))) / (2 * h)
        assert g.numpy()[i] == pytest.approx(numeric, rel=1e-6)


def test_while_loop_newton_and_its_limits():
    def sqrt_newton(a):
        def cond(s):
            return abs(s["x"] * s["x"] - a) > 1e-10

        def body(s):
            return {"x": 0.5 * (s["x"] + a / s["x"]), "n": s["n"] + 1}

        return rg.while_loop(cond, body, {"x": a, "n": rg.tensor(0, "int32")})

    c = rg.compile(sqrt_newton, (f64(2.0),))
    assert c.report["status"] == "ok", c.report
    a, b = c(f64(2.0)), c(f64(1e6))
    assert float(a["x"]) == pytest.approx(2 ** 0.5)
    assert float(b["x"]) == pytest.approx(1e3)
    assert int(b["n"]) > int(a["n"])

    stuck = rg.compile(lambda s: rg.while_loop(lambda v: v < 1e9, lambda v: v, s, max_iterations=5), (f64(1.0),))
    assert stuck.report["diagnostics"][0]["code"] == "WHILE_LIMIT_REACHED"
    with pytest.raises(rg.DiagnosticError) as e:
        rg.grad(lambda v: rg.while_loop(lambda s: s < 10.0, lambda s: s * 2.0, v))(f64(1.0))
    assert e.value.diagnostic["code"] == "GRAD_THROUGH_WHILE"
    with pytest.raises(rg.DiagnosticError) as e:
        rg.while_loop(lambda s: s, lambda s: s, f64([1.0, 2.0]))
    assert e.value.diagnostic["code"] == "CONTROL_FLOW_SHAPE_MISMATCH"


def test_cond_is_lazy_differentiable_and_checks_branches():
    def f(x, flag):
        return rg.cond(flag, lambda v: v.log(), lambda v: v * v, x)

    assert float(f(f64(-3.0), f64(0.0))) == 9.0  # log(-3) never runs
    assert float(rg.grad(f)(f64(2.0), f64(1.0))) == 0.5
    assert float(rg.grad(f)(f64(2.0), f64(0.0))) == 4.0
    good = rg.compile(f, (f64(-3.0), f64(0.0)))
    assert good.report["status"] == "ok", good.report
    bad = good.check(f64(-3.0), f64(1.0))
    assert bad["diagnostics"][0]["diagnosis"]["cause"] == "log_of_negative"

    # Captured outer values in only one branch.
    k = f64(10.0)
    assert float(rg.cond(f64(1.0), lambda v: v + k, lambda v: v, f64(1.0))) == 11.0
    assert float(rg.cond(f64(0.0), lambda v: v, lambda v: v + k, f64(1.0))) == 11.0
    with pytest.raises(rg.DiagnosticError) as e:
        rg.cond(f64(1.0), lambda v: v, lambda v: v.reshape(1), f64(1.0))
    assert e.value.diagnostic["code"] == "CONTROL_FLOW_SHAPE_MISMATCH"


@pytest.mark.parametrize("device", DEVICES)
def test_control_flow_in_the_step_loop(device):
    """`run` over a program whose step holds a scan: the state handoff and history work as for
    any other program (validate.rs:289-363)."""
    def step(state):
        def cell(h, _):
            return rg.tanh(h * state["w"] + 0.1), h.sum()

        h, ys = rg.scan(cell, state["h"], length=6)
        loss = (h * h).sum() + ys.sum()
        return {"h": h, "w": state["w"] * 0.99}, loss

    state = {"h": f64([0.2, -0.1, 0.4]), "w": f64([0.9, 1.1, 0.7])}
    c = rg.compile(step, (state,), device=device)
    r = rg.run(c, state, steps=5)
    h, w, losses = state["h"].numpy(), state["w"].numpy(), []
    for _ in range(5):
        total = 0.0
        for _ in range(6):
            total += h.sum()
            h = np.tanh(h * w + 0.1)
        losses.append((h * h).sum() + total)
        w = w * 0.99
    np.testing.assert_allclose(r.state["h"].numpy(), h, rtol=1e-13)
    np.testing.assert_allclose(np.array(r.history["aux"]), np.array(losses), rtol=1e-13)
