"""Known answers of the engine and the CPU oracle (restating the reference's tests/engine.rs).

Each test builds a graph through the engine, plans it, and executes the plan on the CPU oracle
(oracle/cpu_exec.cpp). Exact values come from the reference's own tests; where a test there
compares with Rust std, this compares with Python's math (the same glibc libm).
"""

import json
import math

import numpy as np
import pytest
import torch

import rustautograd_amd as rg
from helpers import G, diag_code

from conftest import DEVPLAN


def test_broadcasting_and_kernels():
    """engine.rs:47-77: elementwise broadcast, transpose, reductions, slice, pad and matmul values."""
    g = G()
    a = g.const([1., 2., 3., 4., 5., 6.], (2, 3))
    b = g.const([10., 20., 30.])
    c = g.const([100., 200.], (2, 1))
    s = g.scalar(2.0)
    outs = [
        g.bin("add", a, b), g.bin("mul", a, c), g.bin("sub", s, a), g.un("transpose", a, perm=[1, 0]),
        g.op("sum", [a], axes=[0], keepdims=False), g.op("max", [a], axes=[1], keepdims=True),
        g.op("slice", [a], starts=[1, 1], stops=[2, 3]), g.op("pad", [b], starts=[1], shape=[5]), g.bin("matmul", a, b),
    ]
    for device in ("cpu", DEVPLAN):
        r = g.eval(outs, device=device)
        assert r[0].ravel().tolist() == [11., 22., 33., 14., 25., 36.]
        assert r[1].ravel().tolist() == [100., 200., 300., 800., 1000., 1200.]
        assert r[2].ravel().tolist() == [1., 0., -1., -2., -3., -4.]
        assert r[3].shape == (3, 2) and r[3].ravel().tolist() == [1., 4., 2., 5., 3., 6.]
        assert r[4].tolist() == [5., 7., 9.]
        assert r[5].shape == (2, 1) and r[5].ravel().tolist() == [3., 6.]
        assert r[6].ravel().tolist() == [5., 6.]
        assert r[7].tolist() == [0., 10., 20., 30., 0.]
        assert r[8].tolist() == [140., 320.]


def test_static_errors_are_structured():
    """engine.rs:79-90."""
    g = G()
    a = g.const(np.zeros(6), (2, 3))
    b = g.const(np.zeros(2))
    with pytest.raises(rg.DiagnosticError) as e:
        g.bin("add", a, b)
    assert diag_code(e) == "SHAPE_MISMATCH"
    assert e.value.diagnostic["observation"]["lhs_shape"] == [2, 3]
    with pytest.raises(rg.DiagnosticError) as e:
        g.bin("matmul", a, a)
    assert diag_code(e) == "SHAPE_MISMATCH"
    f = g.const(np.zeros(2), dtype="float32")
    with pytest.raises(rg.DiagnosticError) as e:
        g.bin("add", b, f)
    assert diag_code(e) == "DTYPE_MISMATCH"
    with pytest.raises(rg.DiagnosticError) as e:
        g.grad(a, [a])
    assert diag_code(e) == "GRAD_NON_SCALAR"


VJP_CASES = {
    "neg": lambda g, x, w: g.un("neg", x),
    "exp": lambda g, x, w: g.un("exp", x),
    "log": lambda g, x, w: g.un("log", x),
    "sqrt": lambda g, x, w: g.un("sqrt", x),
    "sin": lambda g, x, w: g.un("sin", x),
    "cos": lambda g, x, w: g.un("cos", x),
    "tanh": lambda g, x, w: g.un("tanh", x),
    "abs": lambda g, x, w: g.un("abs", x),
    "add_bcast": lambda g, x, w: g.bin("add", x, w),
    "sub_bcast": lambda g, x, w: g.bin("sub", w, x),
    "mul_bcast": lambda g, x, w: g.bin("mul", x, w),
    "div_bcast": lambda g, x, w: g.bin("div", x, w),
    "div_bcast_rev": lambda g, x, w: g.bin("div", w, x),
    "pow_const": lambda g, x, w: g.bin("pow", x, g.scalar(3.0)),
    "pow_var": lambda g, x, w: g.bin("pow", x, w),
    "pow_exponent": lambda g, x, w: g.bin("pow", w, x),
    "maximum": lambda g, x, w: g.bin("maximum", x, w),
    "minimum": lambda g, x, w: g.bin("minimum", x, w),
    "where": lambda g, x, w: g.op("where", [g.bin("gt", x, w), x, w]),
    "matmul_mv": lambda g, x, w: g.bin("matmul", x, w),
    "matmul_vm": lambda g, x, w: g.bin("matmul", g.const([0.5, -1.0]), x),
    "matmul_mm": lambda g, x, w: (lambda m: g.bin("mul", m, m))(g.bin("matmul", x, g.un("transpose", x, perm=[1, 0]))),
    "reduce_axis": lambda g, x, w: (lambda s: g.bin("mul", s, s))(g.op("sum", [x], axes=[1], keepdims=False)),
    "reduce_max": lambda g, x, w: (lambda s: g.bin("mul", s, s))(g.op("max", [x], axes=[0], keepdims=False)),
    "reduce_min_all": lambda g, x, w: g.op("min", [x], axes=[0, 1], keepdims=False),
    "reshape": lambda g, x, w: (lambda r: g.bin("mul", r, r))(g.un("reshape", x, shape=[3, 2])),
    "transpose": lambda g, x, w: (lambda r: g.bin("mul", r, r))(g.un("transpose", x, perm=[1, 0])),
    "broadcast_to": lambda g, x, w: (lambda r: g.bin("mul", r, r))(g.un("broadcast_to", x, shape=[4, 2, 3])),
    "slice": lambda g, x, w: (lambda r: g.bin("mul", r, r))(g.op("slice", [x], starts=[0, 1], stops=[2, 3])),
    "pad": lambda g, x, w: (lambda r: g.bin("mul", r, r))(g.op("pad", [x], starts=[1, 0], shape=[4, 3])),
}


@pytest.mark.parametrize("name", sorted(VJP_CASES))
def test_every_vjp_matches_finite_differences(name):
    """engine.rs:97-163: analytic gradients in f64 against central differences (h = 1e-6)."""
    x0 = np.array([[0.3, 0.7, 1.1], [1.3, 0.2, 0.9]])
    w0 = np.array([0.5, 1.5, 0.25])
    g = G()
    x, w = g.input((2, 3)), g.input((3,))
    y = g.sum_all(VJP_CASES[name](g, x, w))
    grads = g.grad(y, [x, w])
    fwd = g.compile([y], [x0, w0])
    analytic = g.eval(grads, [x0, w0])
    for which, base in enumerate((x0, w0)):
        for e in range(base.size):
            def probe(d):
                v = base.copy().ravel()
                v[e] += d
                args = [v.reshape(base.shape) if k == which else (x0, w0)[k] for k in range(2)]
                return rg.Tensor(fwd.call([rg.tensor(a)._t for a in args])[0]).numpy().item()
            h = 1e-6
            numeric = (probe(h) - probe(-h)) / (2 * h)
            a = analytic[which].ravel()[e]
            assert abs(a - numeric) < 1e-5 * max(abs(a), 1.0), f"{name} input {which}[{e}]: analytic {a} numeric {numeric}"


def test_higher_order_gradient():
    """engine.rs:165-179: d/dx, d2/dx2, d3/dx3 of x^4 at 2 are 32, 48, 48."""
    g = G()
    x = g.input(())
    y = g.bin("pow", x, g.scalar(4.0))
    d1 = g.grad(y, [x])[0]
    d2 = g.grad(d1, [x])[0]
    d3 = g.grad(d2, [x])[0]
    r = g.eval([d1, d2, d3], [np.array(2.0)])
    assert [v.item() for v in r] == [32.0, 48.0, 48.0]


def test_stop_gradient_and_disconnected():
    """engine.rs:181-190."""
    g = G()
    x, z = g.input(()), g.input(())
    y = g.bin("mul", g.un("stop_gradient", x), x)
    gr = g.grad(y, [x, z])
    r = g.eval(gr, [np.array(3.0), np.array(1.0)])
    assert r[0].item() == 3.0 and r[1].item() == 0.0


def test_optimizer_simplifies_and_keeps_semantics():
    """engine.rs:192-213: folding, simplification and CSE leave input, 4, x*x, *4, add."""
    g = G()
    x = g.input((3,))
    zero, one, two, two_b = g.scalar(0.0), g.scalar(1.0), g.scalar(2.0), g.scalar(2.0)
    b = g.bin("mul", g.bin("add", x, zero), one)
    four = g.bin("add", two, two_b)
    p, q = g.bin("pow", b, two), g.bin("pow", b, two_b)
    g.un("exp", x)
    out = g.bin("add", g.bin("mul", p, four), g.bin("mul", q, four))
    xs = [np.array([1., 2., 3.])]
    c = g.compile([out], xs, optimize="standard", level="standard")
    st = json.loads(c.report_json)["graph"]["optimization"]
    assert st["constants_folded"] >= 1 and st["algebraic_simplified"] >= 3 and st["cse_merged"] >= 1, st
    assert st["nodes_after"] == 5, st
    want = g.eval([out], xs)[0]
    assert rg.Tensor(c.call([rg.tensor(xs[0])._t])[0]).numpy().tolist() == want.tolist() == [8., 32., 72.]


def test_optimizer_never_erases_nan_through_mul_zero():
    """engine.rs:215-224."""
    g = G()
    x = g.input(())
    out = g.bin("mul", x, g.scalar(0.0))
    assert math.isnan(g.eval([out], [np.array(np.nan)], optimize="standard")[0].item())


TRANSPOSE_CASES = [
    lambda g, a, b, c, v: g.bin("matmul", g.un("transpose", a, perm=[1, 0]), b),
    lambda g, a, b, c, v: g.bin("matmul", a, g.un("transpose", b, perm=[1, 0])),
    lambda g, a, b, c, v: g.bin("matmul", a, g.un("transpose", c, perm=[1, 0])),
    lambda g, a, b, c, v: g.bin("matmul", g.un("transpose", c, perm=[1, 0]), g.un("transpose", a, perm=[1, 0])),
    lambda g, a, b, c, v: g.bin("matmul", g.un("transpose", a, perm=[1, 0]), v),
]


@pytest.mark.parametrize("k", range(len(TRANSPOSE_CASES)))
def test_transposed_matmul_rewrite_covers_every_flag_combination(k):
    """engine.rs:327-362: transposes feeding a product become MatMulT flags, results unchanged."""
    a = np.array([[1., 2., 3.], [4., 5., 6.]])
    b = np.array([[7., 8., 9.], [10., 11., 12.]])
    c = np.array([[1., 0., 2.], [0., 3., 0.], [4., 0., 5.]])
    v = np.array([0.5, -2.0])
    g = G()
    ids = g.input((2, 3)), g.input((2, 3)), g.input((3, 3)), g.input((2,))
    out = TRANSPOSE_CASES[k](g, *ids)
    args = [a, b, c, v]
    want = g.eval([out], args)[0]
    for device in ("cpu", DEVPLAN):
        comp = g.compile([out], args, device=device, optimize="standard")
        plan = comp.plan_summary()
        assert not any(s.get("op") == "transpose" for s in plan), f"case {k} kept a transpose copy"
        assert any(s.get("op") == "matmul_t" for s in plan), f"case {k} was not rewritten"
        got = rg.Tensor(comp.call([rg.tensor(x)._t for x in args])[0]).numpy()
        assert got.tolist() == want.tolist()
    np.testing.assert_allclose(want, TRANSPOSE_NUMPY[k](a, b, c, v), rtol=0, atol=0)


TRANSPOSE_NUMPY = [
    lambda a, b, c, v: a.T @ b, lambda a, b, c, v: a @ b.T, lambda a, b, c, v: a @ c.T,
    lambda a, b, c, v: c.T @ a.T, lambda a, b, c, v: a.T @ v,
]


def test_transpose_with_another_consumer_survives():
    """engine.rs:354-361."""
    a = np.array([[1., 2., 3.], [4., 5., 6.]])
    g = G()
    x = g.input((2, 3))
    tx = g.un("transpose", x, perm=[1, 0])
    m = g.bin("matmul", tx, x)
    r = g.eval([m, tx], [a], optimize="standard")
    assert r[0].tolist() == (a.T @ a).tolist() and r[1].tolist() == a.T.tolist()


def test_groups_form_and_results_ignore_thread_count(oracle_threads):
    """engine.rs:439-471: one fused group of 4 ops; only its output needs a buffer; thread invariance."""
    g = G()
    x = g.input((1000, 64), "float32")
    b = g.input((64,), "float32")
    h = g.un("tanh", g.bin("add", x, b))
    e = g.un("exp", g.bin("mul", h, h))
    xs = np.sin(np.arange(64000) * 0.37).reshape(1000, 64).astype(np.float32)
    bs = (np.arange(64) * 0.01).astype(np.float32)
    c = g.compile([e], [xs, bs], device=DEVPLAN)
    fused = [s for s in c.plan_summary() if s["kind"] == "fused"]
    assert len(fused) == 1 and len(fused[0]["ops"]) == 4
    assert fused[0]["input_kinds"] == ["full", "row"]
    mem = json.loads(c.report_json)["memory"]
    assert mem["intermediate_bytes_planned"] == 64000 * 4
    assert mem["intermediate_bytes_without_reuse"] == 4 * 64000 * 4
    cpu = g.compile([e], [xs, bs])
    runs = []
    for threads in (1, 2, 7):
        oracle_threads(threads)
        runs.append(rg.Tensor(cpu.call([rg.tensor(xs)._t, rg.tensor(bs)._t])[0]).numpy())
    assert all(np.array_equal(runs[0], r) for r in runs[1:])
    want = np.exp(np.tanh(xs.astype(np.float64) + bs) ** 2)
    np.testing.assert_allclose(runs[0], want, rtol=1e-6)


def test_memory_plan_reuses_buffers_and_works_in_place():
    """engine.rs:477-489: twenty chained sines reuse one buffer."""
    g = G()
    x = g.input((1000,))
    v = x
    for _ in range(20):
        v = g.un("sin", v)
    mem = json.loads(g.compile([v], [np.zeros(1000)]).report_json)["memory"]
    assert mem["intermediate_bytes_without_reuse"] == 20 * 8000
    assert mem["intermediate_bytes_planned"] == 8000


@pytest.mark.parametrize("name,ref", [("exp", math.exp), ("log", math.log), ("sin", math.sin), ("cos", math.cos), ("tanh", math.tanh)])
def test_vector_math_in_place_matches_libm(name, ref):
    """engine.rs:491-518: per-element libm in place, 1500 elements across block boundaries."""
    v = 0.001 + np.arange(1500) * 0.01
    g = G()
    x = g.input((1500,))
    scaled = g.bin("mul", x, g.scalar(0.5))
    out = g.un(name, scaled)
    c = g.compile([out], [v])
    steps = [s for s in c.plan_summary() if s["kind"] == "instr"]
    assert steps[1]["dst"] == steps[1]["args"][0], f"{name} must run in place"
    got = rg.Tensor(c.call([rg.tensor(v)._t])[0]).numpy()
    want = np.array([ref(b * 0.5) for b in v])
    assert np.all(np.abs(got - want) <= 1e-14 * np.maximum(np.abs(want), 1.0))


def test_log_ieee_edges():
    """engine.rs:511-517."""
    g = G()
    x = g.input((4,))
    r = g.eval([g.un("log", x)], [np.array([-1.0, 0.0, np.inf, np.nan])])[0]
    assert np.isnan(r[0]) and r[1] == -np.inf and r[2] == np.inf and np.isnan(r[3])


def test_f32_precision_is_real():
    """engine.rs:747-753: float32 programs compute in float32."""
    g = G()
    x = g.input((2,), "float32")
    r = g.eval([g.bin("add", x, x)], [np.array([0.1, 0.2], np.float32)])[0]
    assert r.dtype == np.float32 and r.tolist() == [np.float32(0.2), np.float32(0.4)]


def test_take_concat_argmax_and_int_arithmetic():
    """engine.rs:760-785."""
    g = G()
    x = g.const([1., 2., 3., 4., 5., 6.], (3, 2))
    idx = g.const([2, 0, 1, 1], (2, 2), "int32")
    col = g.const([1], (1,), "int32")
    along = g.const([1, 0, 1], (3, 1), "int32")
    outs = [g.op("take", [x, idx], axis=0), g.op("take", [x, col], axis=1), g.op("take_along", [x, along]),
            g.op("concat", [x, x], axis=1), g.op("argmax", [x]), g.bin("add", col, g.const(1, (), "int32"))]
    for device in ("cpu", DEVPLAN):
        r = g.eval(outs, device=device)
        assert r[0].shape == (2, 2, 2) and r[0].ravel().tolist() == [5., 6., 1., 2., 3., 4., 3., 4.]
        assert r[1].ravel().tolist() == [2., 4., 6.]
        assert r[2].ravel().tolist() == [2., 3., 6.]
        assert r[3].ravel().tolist() == [1., 2., 1., 2., 3., 4., 3., 4., 5., 6., 5., 6.]
        assert r[4].dtype == np.int32 and r[4].tolist() == [1, 1, 1]
        assert r[5].dtype == np.int32 and r[5].tolist() == [2]
    with pytest.raises(rg.DiagnosticError) as e:
        g.un("exp", col)
    assert diag_code(e) == "UNSUPPORTED_DTYPE"
    with pytest.raises(rg.DiagnosticError) as e:
        g.op("take", [x, x], axis=0)
    assert diag_code(e) == "DTYPE_MISMATCH"


def _ints(g, values, shape):
    return g.const(values, shape, "int32")


NEW_OP_CASES = {
    "take_embedding": lambda g, x: (lambda r: g.bin("mul", r, r))(g.op("take", [x, _ints(g, [1, 0, 1, 1, 0, 0], (3, 2))], axis=0)),
    "take_axis2": lambda g, x: (lambda r: g.bin("mul", r, r))(g.op("take", [x, _ints(g, [3, 3], (2,))], axis=2)),
    "take_along": lambda g, x: g.un("log", g.op("take_along", [x, _ints(g, [0, 3, 1, 1, 2, 0, 3, 3, 0, 1, 2, 2], (2, 3, 2))])),
    "concat": lambda g, x: (lambda r: g.bin("mul", r, r))(g.op("concat", [x, g.un("exp", x), x], axis=1)),
    "batched_matmul": lambda g, x: (lambda m: g.bin("mul", m, m))(g.bin("matmul", x, g.un("transpose", x, perm=[0, 2, 1]))),
    "batched_broadcast": lambda g, x: (lambda m: g.bin("mul", m, m))(g.bin("matmul", x, g.const([0.5, 1., -1., 2., 3., 0.25, 1., 1.], (4, 2)))),
    "rhs_batched": lambda g, x: (lambda m: g.bin("mul", m, m))(g.bin("matmul", g.const(np.arange(15) * 0.1, (5, 3)), x)),
    "vector_rhs": lambda g, x: (lambda m: g.bin("mul", m, m))(g.bin("matmul", x, g.const([1., 2., 3., 4.]))),
    "vector_lhs": lambda g, x: (lambda m: g.bin("mul", m, m))(g.bin("matmul", g.const([1., 2., 3.]), x)),
    "floor_blocks": lambda g, x: g.bin("mul", g.un("floor", x), x),
}


@pytest.mark.parametrize("name", sorted(NEW_OP_CASES))
def test_new_op_gradients_match_finite_differences(name):
    """engine.rs:787-826: gather, scatter, concat and batched-product gradients, plain and device-planned."""
    x0 = (0.1 + np.sin(np.arange(24) * 0.7) * 0.4 + 0.5).reshape(2, 3, 4)
    g = G()
    x = g.input((2, 3, 4))
    y = g.sum_all(NEW_OP_CASES[name](g, x))
    gx = g.grad(y, [x])[0]
    analytic = g.eval([gx], [x0])[0].ravel()
    planned = g.eval([gx], [x0], device=DEVPLAN, optimize="standard")[0].ravel()
    fwd = g.compile([y], [x0])
    for e in range(x0.size):
        def probe(d):
            v = x0.copy().ravel()
            v[e] += d
            return rg.Tensor(fwd.call([rg.tensor(v.reshape(x0.shape))._t])[0]).numpy().item()
        numeric = (probe(1e-6) - probe(-1e-6)) / 2e-6
        assert abs(analytic[e] - numeric) < 1e-4 * max(abs(analytic[e]), 1.0), f"{name}[{e}]: {analytic[e]} vs {numeric}"
        assert abs(analytic[e] - planned[e]) < 1e-9 * max(abs(analytic[e]), 1.0), f"{name}[{e}] device plan"


def test_second_order_through_take():
    """engine.rs:828-843: f = sum(x[idx]^3) with repeats; f'' along the diagonal is 6*x*count."""
    g = G()
    x = g.input((3,))
    tk = g.op("take", [x, _ints(g, [0, 2, 2, 1], (4,))], axis=0)
    y = g.sum_all(g.bin("pow", tk, g.scalar(3.0)))
    g1 = g.grad(y, [x])[0]
    g2 = g.grad(g.sum_all(g1), [x])[0]
    for device in ("cpu", DEVPLAN):
        assert g.eval([g2], [np.array([1., 2., 3.])], device=device)[0].tolist() == [6., 12., 36.]


def test_out_of_range_index_is_clamped_and_a_validation_error():
    """engine.rs:892-904."""
    g = G()
    x = g.input((3,))
    o = g.op("take", [x, _ints(g, [5, -1], (2,))], axis=0)
    x0 = np.array([1., 2., 3.])
    assert g.eval([o], [x0])[0].tolist() == [3., 1.]
    rep = json.loads(g.compile([o], [x0], level="standard").report_json)
    assert rep["status"] == "validation_failed"
    assert rep["diagnostics"][0]["code"] == "INDEX_OUT_OF_RANGE"
    assert rep["diagnostics"][0]["observation"]["index_max"] == 5.0


def test_parallel_structural_kernels_ignore_thread_count(oracle_threads):
    """engine.rs:945-977: transposes and reductions above the parallel thresholds; hand references."""
    a, b, c = 128, 100, 100
    xs = np.sin(np.arange(a * b * c) * 0.37)
    x0 = xs.reshape(a, b, c).astype(np.float32)
    g = G()
    x = g.input((a, b, c), "float32")
    outs = [g.un("transpose", x, perm=[2, 0, 1]), g.un("transpose", x, perm=[1, 0, 2]),
            g.op("max", [x], axes=[2], keepdims=True), g.op("sum", [x], axes=[2], keepdims=False),
            g.op("sum", [x], axes=[0, 1], keepdims=True), g.op("min", [x], axes=[0, 1], keepdims=False)]
    comp = g.compile(outs, [x0])
    runs = []
    for threads in (1, 3, 8):
        oracle_threads(threads)
        runs.append([rg.Tensor(t).numpy() for t in comp.call([rg.tensor(x0)._t])])
    for r in runs[1:]:
        assert all(np.array_equal(p, q) for p, q in zip(runs[0], r))
    one = runs[0]
    flat = x0.reshape(a * b, c)
    for ci in (0, 7, c - 1):
        assert abs(one[4].ravel()[ci] - flat[:, ci].astype(np.float64).sum()) < 1e-2
        assert one[5][ci] == flat[:, ci].min()
    row = 5 * b + 3
    assert one[2].ravel()[row] == flat[row].max()
    assert one[0].shape == (c, a, b)
    assert one[0].ravel()[a * b + 2] == x0[0, 2, 1]
    np.testing.assert_array_equal(one[1], x0.transpose(1, 0, 2))


def test_arg_top_k_orders_ties_and_nan_deterministically():
    """engine.rs:1315-1326: descending, ties by lower index, NaN ranked highest; k > axis rejected."""
    g = G()
    x = g.input((2, 5))
    k2 = g.op("arg_top_k", [x], k=2)
    k5 = g.op("arg_top_k", [x], k=5)
    v = np.array([1.0, 3.0, 2.0, 3.0, 0.0, np.nan, -1.0, np.nan, 4.0, 2.0]).reshape(2, 5)
    r = g.eval([k2, k5], [v])
    assert r[0].dtype == np.int32 and r[0].ravel().tolist() == [1, 3, 3, 4]
    assert r[1].ravel().tolist() == [1, 3, 2, 0, 4, 3, 4, 1, 0, 2]
    with pytest.raises(rg.DiagnosticError) as e:
        g.op("arg_top_k", [x], k=6)
    assert diag_code(e) == "INVALID_AXIS"


def test_large_top_k_ignores_thread_count(oracle_threads):
    """engine.rs:1328-1338."""
    n = 1 << 18
    v = np.round(np.sin((np.arange(n) * 37 % 1000) * 0.73)).reshape(n // 64, 64)
    g = G()
    x = g.input(v.shape)
    c = g.compile([g.op("arg_top_k", [x], k=9)], [v])
    oracle_threads(1)
    serial = rg.Tensor(c.call([rg.tensor(v)._t])[0]).numpy()
    oracle_threads(8)
    assert np.array_equal(serial, rg.Tensor(c.call([rg.tensor(v)._t])[0]).numpy())
    # numpy's stable argsort of -v orders ties by index; NaN is absent here.
    np.testing.assert_array_equal(serial, np.argsort(-v, axis=1, kind="stable")[:, :9])


def test_cumsum_and_its_gradient():
    """engine.rs:1340-1356."""
    g = G()
    x = g.input((2, 3))
    c = g.op("cumsum", [x], reverse=False)
    r = g.op("cumsum", [x], reverse=True)
    y = g.sum_all(g.bin("mul", c, g.const([1., 10., 100., 2., 20., 200.], (2, 3))))
    gx = g.grad(y, [x])[0]
    out = g.eval([c, r, gx], [np.array([[1., 2., 3.], [4., 5., 6.]])])
    assert out[0].ravel().tolist() == [1., 3., 6., 4., 9., 15.]
    assert out[1].ravel().tolist() == [6., 5., 3., 15., 11., 6.]
    assert out[2].ravel().tolist() == [111., 110., 100., 222., 220., 200.]


def _optimal_chain_flops(d):
    """The textbook matrix-chain dynamic program (engine.rs:1375-1386)."""
    n = len(d) - 1
    m = [[0.0] * n for _ in range(n)]
    for length in range(2, n + 1):
        for i in range(n - length + 1):
            j = i + length - 1
            m[i][j] = min(m[i][k] + m[k + 1][j] + d[i] * d[k + 1] * d[j + 1] for k in range(i, j))
    return m[0][n - 1]


@pytest.mark.parametrize("sizes", [[30, 35, 15, 5, 10, 20, 25], [1024, 8, 1024, 8, 1024], [4, 300, 2, 500, 3, 200, 6], [10, 20, 30, 40, 30]])
def test_search_finds_the_optimal_matrix_chain_order(sizes):
    """engine.rs:1393-1411: the extracted chain costs at most 1% above the DP optimum (CPU model)."""
    from rustautograd_amd import _rg
    g = G()
    ids, inputs = [], []
    for a, b in zip(sizes, sizes[1:]):
        ids.append(g.input((a, b)))
        inputs.append(np.sin(np.arange(a * b) * 0.31).reshape(a, b))
    v = ids[0]
    for m in ids[1:]:
        v = g.bin("matmul", v, m)
    products = _rg.matrix_search_products(g.g, [v], False)
    if products is None:
        products = [(sizes[0], sizes[k], sizes[k + 1]) for k in range(1, len(sizes) - 1)]
    flops = sum(m * k * n for m, k, n in products)
    best = _optimal_chain_flops(sizes)
    assert flops <= best * 1.01, f"{sizes}: {flops} multiplications, optimal is {best}"
    want = inputs[0]
    for m in inputs[1:]:
        want = want @ m
    for mode in ("search-linear", "search"):
        c = g.compile([v], inputs, optimize=mode)
        got = rg.Tensor(c.call([rg.tensor(x)._t for x in inputs])[0]).numpy()
        assert np.abs(got - want).max() <= 1e-9 * max(1.0, np.abs(want).max())


def test_compile_reorders_matrix_products_by_default_and_can_be_told_not_to():
    """test_framework.py:705-729, on the Python surface."""
    r = np.random.default_rng(10)
    a, b, c, x = r.normal(size=(256, 4)), r.normal(size=(4, 256)), r.normal(size=(256, 4)), r.normal(size=(4,))
    f = lambda a, b, c, x: ((a @ b @ c) @ x).sum()
    inputs = tuple(rg.tensor(v) for v in (a, b, c, x))
    default = rg.compile(f, inputs, validate="thorough")
    plain = rg.compile(f, inputs, validate="thorough", optimize="standard")
    search = default.report["graph"]["optimization"]["search"]
    assert search["accepted"] and search["cost_after"] < search["cost_before"] * 0.5
    assert plain.report["graph"]["optimization"]["search"] is None
    assert default.report["status"] == "ok", default.report
    assert float(default(*inputs)) == pytest.approx(float(plain(*inputs)), rel=1e-11)
    assert float(rg.compile(f, inputs, optimize="auto")(*inputs)) == pytest.approx(float(plain(*inputs)), rel=1e-11)
    with pytest.raises(ValueError):
        rg.compile(f, inputs, optimize="magic")
    fn = rg.grad(f, argnums=(0, 3))
    ga, gx = rg.compile(fn, inputs)(*inputs)
    pa, px = rg.compile(fn, inputs, optimize="standard")(*inputs)
    np.testing.assert_allclose(ga.numpy(), pa.numpy(), rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(gx.numpy(), px.numpy(), rtol=1e-10, atol=1e-11)
    # An independent check of the value: numpy in f64.
    assert float(default(*inputs)) == pytest.approx(float(((a @ b @ c) @ x).sum()), rel=1e-10)


def test_exact_rules_never_change_a_bit_on_special_values():
    """engine.rs:1439-1464."""
    sp = [0.0, -0.0, 1.0, -1.5, 1e300, -1e300, np.inf, -np.inf, np.nan, 1e-300]
    n = len(sp)
    a = np.repeat(sp, n)
    b = np.tile(sp, n)
    g = G()
    x, y = g.input((n * n,)), g.input((n * n,))
    nx = g.un("neg", x)
    outs = [g.bin("sub", g.un("neg", nx), y), g.bin("mul", nx, y), g.bin("div", nx, y), g.bin("add", y, x)]
    want = g.eval(outs, [a, b])
    for mode in ("search-exact", "standard"):
        got = g.eval(outs, [a, b], optimize=mode)
        for u, v in zip(want, got):
            assert np.array_equal(u.view(np.int64), v.view(np.int64)) or np.array_equal(u, v, equal_nan=True)


def test_row_parallel_checker_gemm_is_bit_identical_to_the_serial_loop():
    """The oracle's optional row split of 2-D products keeps every element's summation order."""
    import ctypes
    from conftest import ORACLE
    lib = ctypes.CDLL(ORACLE)
    r = np.random.default_rng(1)
    a = r.normal(size=(3, 300, 256)).astype(np.float32)
    b = r.normal(size=(256, 200)).astype(np.float32)
    g = G()
    x, w = g.input(a.shape, "float32"), g.input(b.shape, "float32")
    c = g.compile([g.bin("matmul", x, w)], [a, b])
    args = [rg.tensor(a)._t, rg.tensor(b)._t]
    try:
        lib.rg_cpu_set_row_parallel_gemm(0)
        serial = rg.Tensor(c.call(args)[0]).numpy()
        lib.rg_cpu_set_row_parallel_gemm(1)
        parallel = rg.Tensor(c.call(args)[0]).numpy()
    finally:
        lib.rg_cpu_set_row_parallel_gemm(1)
    assert np.array_equal(serial.view(np.int32), parallel.view(np.int32))
    np.testing.assert_allclose(serial, a.astype(np.float64) @ b, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_blocked_checker_gemm_is_bit_identical_for_every_transpose_flag(ta, tb):
    """The checker's blocked products (stacked rows, single large products such as the weight
    gradients, transposed operands through a copied panel) add each output's terms in the
    serial loop's order: every flag combination gives the serial loop's bits."""
    import ctypes
    from conftest import ORACLE
    lib = ctypes.CDLL(ORACLE)
    r = np.random.default_rng(2)
    m, k, n = 150, 333, 290
    a = r.normal(size=(k, m) if ta else (m, k)).astype(np.float32)
    b = r.normal(size=(n, k) if tb else (k, n)).astype(np.float32)
    g = G()
    x, w = g.input(a.shape, "float32"), g.input(b.shape, "float32")
    lhs = g.un("transpose", x, perm=[1, 0]) if ta else x
    rhs = g.un("transpose", w, perm=[1, 0]) if tb else w
    c = g.compile([g.bin("matmul", lhs, rhs)], [a, b], optimize="standard")
    assert any(st.get("op") == "matmul_t" for st in c.plan_summary()) == (ta or tb)
    args = [rg.tensor(a)._t, rg.tensor(b)._t]
    try:
        lib.rg_cpu_set_row_parallel_gemm(0)
        serial = rg.Tensor(c.call(args)[0]).numpy()
        lib.rg_cpu_set_row_parallel_gemm(1)
        blocked = rg.Tensor(c.call(args)[0]).numpy()
    finally:
        lib.rg_cpu_set_row_parallel_gemm(1)
    assert np.array_equal(serial.view(np.int32), blocked.view(np.int32))
    want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b)
    np.testing.assert_allclose(serial, want, rtol=1e-4, atol=1e-4)


def test_where_with_broadcast_operand_differentiates_in_a_growing_graph():
    """Regression: the gradient of where() through a broadcast operand, built while the node table
    reallocates (unbroadcast once read its target shape through a reference into that table)."""
    g = G()
    x = g.input((300, 7))
    t = g.un("tanh", x)
    for _ in range(40):  # unrelated nodes, so the table grows during grad
        t = g.un("sin", t)
    a = g.op("sum", [x], axes=[1], keepdims=True)
    w = g.op("where", [g.bin("gt", a, x), a, x])
    gx = g.grad(g.sum_all(w), [x])[0]
    x0 = 0.2 + np.abs(np.sin(np.arange(2100) * 0.37)).reshape(300, 7)
    got = g.eval([gx], [x0])[0]
    xt = torch.tensor(x0, requires_grad=True)
    at = xt.sum(1, keepdim=True)
    torch.where(at > xt, at, xt).sum().backward()
    np.testing.assert_allclose(got, xt.grad.numpy(), rtol=1e-12)


def _plan_ops(g, outs, inputs, device, optimize="standard"):
    return [s["op"] if s["kind"] == "instr" else s["kind"] for s in g.compile(outs, inputs, device, optimize).plan_summary()]


def test_whole_slices_and_in_order_gathers_are_their_input():
    """A slice of the whole value and a gather at constant indices 0..n-1 along an axis of length
    n (a position table read at arange(n)) are the value itself: no step, the same bits."""
    g = G()
    table = g.input((6, 5), "float32")
    x = g.input((6, 5), "float32")
    rows = g.op("take", [table, g.const(np.arange(6), dtype="int32")], axis=0)
    whole = g.op("slice", [x], starts=[0, 0], stops=[6, 5])
    part = g.op("slice", [x], starts=[1, 0], stops=[6, 5])
    y = g.un("tanh", g.bin("add", rows, whole))
    inputs = [np.linspace(-1, 1, 30, dtype=np.float32).reshape(6, 5), np.cos(np.arange(30, dtype=np.float32)).reshape(6, 5)]
    for device in ("cpu", DEVPLAN):
        ops = _plan_ops(g, [y, part], inputs, device)
        assert "take" not in ops and ops.count("slice") == 1, (device, ops)
        got = g.eval([y, part], inputs, device=device, optimize="standard")
        want = g.eval([y, part], inputs, device="cpu", optimize="none")
        for a, b in zip(got, want):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # A permuted or partial index set stays a gather.
    h = G()
    t2 = h.input((6, 5), "float32")
    perm = h.op("take", [t2, h.const(np.array([1, 0, 2, 3, 4, 5]), dtype="int32")], axis=0)
    assert "take" in _plan_ops(h, [perm], inputs[:1], "cpu")


def test_device_plans_merge_equal_constants_beyond_the_reference_limit():
    """Two equal 8 x 8 constants (64 values, above the 16 the reference merges) feeding the same
    product: one product on device plans, the same values; CPU plans keep the reference's limit."""
    g = G()
    d = g.input((40, 8), "float32")
    ones_a = g.const(np.ones((8, 8)), dtype="float32")
    ones_b = g.const(np.ones((8, 8)), dtype="float32")
    p1 = g.op("matmul", [ones_a, g.op("transpose", [d], perm=[1, 0])])
    p2 = g.op("matmul", [ones_b, g.op("transpose", [d], perm=[1, 0])])
    out = g.bin("add", p1, p2)
    inputs = [np.sin(np.arange(320, dtype=np.float32)).reshape(40, 8)]
    dev = _plan_ops(g, [out], inputs, DEVPLAN)
    cpu = _plan_ops(g, [out], inputs, "cpu")
    products = ("matmul", "matmul_t")
    assert sum(o in products for o in dev) == 1 and sum(o in products for o in cpu) == 2, (dev, cpu)
    a = g.eval([out], inputs, device=DEVPLAN, optimize="standard")[0]
    b = g.eval([out], inputs, device="cpu", optimize="none")[0]
    np.testing.assert_allclose(a, b, rtol=1e-6)
