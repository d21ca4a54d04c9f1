"""Row groups in device plans, on the CPU oracle.

The HIP planner fuses a last-axis reduction with the row-wise work around it into a row group,
and folds into the same group the reductions over every other axis (column reductions) of values
it walks, such as a layer norm's scale and shift gradients. The oracle runs a device plan
("cpu_devplan") with the operations of the nodes it replaces; a row group folds each row in
element order (the CPU plan's eight-lane order differs by rounding), and a column reduction
exactly as the standalone reduction it replaces. Results agree with the unfused CPU plan to
rounding (1e-5 relative).
"""

import json

import numpy as np
import pytest

from conftest import DEVPLAN
from helpers import G
from test_hip_rows import _layer_norm


def _plans(g, outs, inputs):
    dev = g.compile(outs, inputs, device=DEVPLAN, optimize="standard")
    cpu = g.compile(outs, inputs, device="cpu", optimize="standard")
    return dev, cpu


@pytest.mark.parametrize("shape", [(64, 256), (3, 40, 96), (9, 7)])
def test_layer_norm_parameter_gradients_fold_into_the_backward_row_group(shape):
    d = shape[-1]
    r = np.random.default_rng(d)
    xv = r.normal(size=shape).astype(np.float32)
    sv = (1 + 0.1 * r.normal(size=d)).astype(np.float32)
    bv = (0.1 * r.normal(size=d)).astype(np.float32)
    wv = r.normal(size=shape).astype(np.float32)
    g = G()
    x, s, b, w = g.input(shape, "float32"), g.input((d,), "float32"), g.input((d,), "float32"), g.input(shape, "float32")
    y = _layer_norm(g, x, s, b, d)
    loss = g.sum_all(g.bin("mul", y, w))
    gx, gs, gb = g.grad(loss, [x, s, b])
    outs, inputs = [y, gx, gs, gb], [xv, sv, bv, wv]
    dev, cpu = _plans(g, outs, inputs)
    steps = dev.plan_summary()
    assert sum(st.get("column_reductions", 0) for st in steps if st["kind"] == "fused") == 2, steps
    assert not any(st["kind"] == "instr" and st["op"] == "sum" for st in steps), [st.get("op") for st in steps]
    a = g.eval(outs, inputs, device=DEVPLAN, optimize="standard")
    b2 = g.eval(outs, inputs, device="cpu", optimize="standard")
    for k, (u, v) in enumerate(zip(a, b2)):
        np.testing.assert_allclose(u, v, rtol=1e-5, atol=1e-5 * np.abs(v).max(), err_msg=f"output {k}")


def test_column_reduction_of_a_value_computed_after_the_group_stays_outside():
    """A reduction whose value depends on the group's result through another reduction cannot
    join it (the fold would need the finished group)."""
    r = np.random.default_rng(3)
    xv = r.normal(size=(32, 64)).astype(np.float32)
    g = G()
    x = g.input((32, 64), "float32")
    m = g.op("max", [x], axes=[1], keepdims=True)
    e = g.un("exp", g.bin("sub", x, m))
    tot = g.op("sum", [e], axes=[0, 1], keepdims=True)  # every axis: a full reduction, not a column one
    z = g.bin("div", e, tot)
    col = g.op("sum", [z], axes=[0], keepdims=False)
    outs, inputs = [col], [xv]
    a = g.eval(outs, inputs, device=DEVPLAN, optimize="standard")
    b = g.eval(outs, inputs, device="cpu", optimize="standard")
    np.testing.assert_allclose(a[0], b[0], rtol=1e-5, atol=1e-5 * np.abs(b[0]).max())


def test_rematerialized_copies_merge_with_their_originals_in_device_plans():
    """An activation kept for the backward pass is rematerialized (a clone with the same inputs)
    while its original still feeds the forward pass; level-order device plans would compute both
    in one group and write the value twice, so device plans merge identical nodes afterwards.
    The CPU plan keeps the clone. Results agree to rounding."""
    r = np.random.default_rng(7)
    xv = r.normal(size=(64, 128)).astype(np.float32)
    w1v = (0.1 * r.normal(size=(128, 512))).astype(np.float32)
    bv = (0.1 * r.normal(size=(512,))).astype(np.float32)
    w2v = (0.1 * r.normal(size=(512, 128))).astype(np.float32)
    tv = r.normal(size=(64, 128)).astype(np.float32)
    g = G()
    x, w1, b, w2, t = (g.input(v.shape, "float32") for v in (xv, w1v, bv, w2v, tv))
    u = g.bin("add", g.op("matmul", [x, w1]), b)
    a = g.bin("mul", u, g.un("tanh", u))  # an activation the backward pass needs
    y = g.op("matmul", [a, w2])
    loss = g.sum_all(g.bin("mul", y, t))
    gw1, gb, gw2 = g.grad(loss, [w1, b, w2])
    outs, inputs = [y, gw1, gb, gw2], [xv, w1v, bv, w2v, tv]
    dev, cpu = _plans(g, outs, inputs)
    st_dev = json.loads(dev.report_json)["graph"]["optimization"]
    st_cpu = json.loads(cpu.report_json)["graph"]["optimization"]
    assert st_cpu["rematerialized"] >= 1, st_cpu
    assert st_dev["cse_merged"] > st_cpu["cse_merged"], (st_dev, st_cpu)
    assert st_dev["nodes_after"] < st_cpu["nodes_after"], (st_dev, st_cpu)
    got = g.eval(outs, inputs, device=DEVPLAN, optimize="standard")
    want = g.eval(outs, inputs, device="cpu", optimize="standard")
    for k, (p, q) in enumerate(zip(got, want)):
        np.testing.assert_allclose(p, q, rtol=1e-5, atol=1e-5 * np.abs(q).max(), err_msg=f"output {k}")


@pytest.mark.parametrize("shape", [(64, 256), (3, 40, 96)])
def test_layer_norm_backward_recomputes_the_forward_rows(shape):
    """The backward row group of a layer norm recomputes the centred input and the normalised
    values (with the row mean and variance) from the input it reads anyway, so the forward row
    group writes only its output; results agree with the CPU plan to rounding."""
    d = shape[-1]
    r = np.random.default_rng(d + 1)
    xv = r.normal(size=shape).astype(np.float32)
    sv = (1 + 0.1 * r.normal(size=d)).astype(np.float32)
    bv = (0.1 * r.normal(size=d)).astype(np.float32)
    wv = r.normal(size=shape).astype(np.float32)
    g = G()
    x, s, b, w = g.input(shape, "float32"), g.input((d,), "float32"), g.input((d,), "float32"), g.input(shape, "float32")
    y = _layer_norm(g, x, s, b, d)
    loss = g.sum_all(g.bin("mul", y, w))
    gx, gs, gb = g.grad(loss, [x, s, b])
    outs, inputs = [y, gx, gs, gb], [xv, sv, bv, wv]
    dev, _ = _plans(g, outs, inputs)
    rows = [st for st in dev.plan_summary() if st["kind"] == "fused" and st["row_len"]]
    assert len(rows) == 2, rows
    assert rows[0]["n_outputs"] == 1, rows[0]
    a = g.eval(outs, inputs, device=DEVPLAN, optimize="standard")
    b2 = g.eval(outs, inputs, device="cpu", optimize="standard")
    for k, (u, v) in enumerate(zip(a, b2)):
        np.testing.assert_allclose(u, v, rtol=1e-5, atol=1e-5 * np.abs(v).max(), err_msg=f"output {k}")


@pytest.mark.parametrize("m,k,n,ta", [(64, 32, 48, False), (40, 24, 16, True)])
def test_bias_adds_fold_into_the_product(m, k, n, ta):
    """A group that only adds a bias vector to the rows of the product before it (its only reader)
    becomes the product's third operand in device plans; the oracle adds it to the finished
    product, so results equal the CPU plan's exactly."""
    r = np.random.default_rng(m + k + n)
    av = r.normal(size=(k, m) if ta else (m, k)).astype(np.float32)
    wv = r.normal(size=(k, n)).astype(np.float32)
    bv = r.normal(size=(n,)).astype(np.float32)
    g = G()
    a, w, b = g.input(av.shape, "float32"), g.input(wv.shape, "float32"), g.input(bv.shape, "float32")
    x = g.op("transpose", [a], perm=[1, 0]) if ta else a
    y = g.bin("add", g.op("matmul", [x, w]), g.op("broadcast_to", [b], shape=[m, n]))
    outs, inputs = [y], [av, wv, bv]
    dev, _ = _plans(g, outs, inputs)
    steps = dev.plan_summary()
    prods = [st for st in steps if st["kind"] == "instr" and st["op"] in ("matmul", "matmul_t")]
    assert len(prods) == 1 and len(prods[0]["args"]) == 3, steps
    got = g.eval(outs, inputs, device=DEVPLAN, optimize="standard")[0]
    want = g.eval(outs, inputs, device="cpu", optimize="standard")[0]
    np.testing.assert_array_equal(got, want)
