"""Row groups on the device: last-axis reductions fused with the work around them.

The HIP planner turns normalisation, softmax, cross-entropy and their backward forms into row
groups (one kernel each: a wavefront per row, the row in registers, wave-shuffle reductions).
These tests run such programs on the device and on the CPU oracle's plan (the reference
interpreter's order) and compare: reductions and what follows them within 1e-4 relative to the
largest magnitude, as for any reduction.
"""

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import nn
from helpers import G, close

from test_plan_fuzz import Twin, XorShift, _row_program

pytestmark = pytest.mark.gpu


def _both(g, outs, inputs, tol=1e-4, what=""):
    hip = g.eval(outs, inputs, device="hip", optimize="standard")
    cpu = g.eval(outs, inputs, device="cpu", optimize="standard")
    for k, (a, b) in enumerate(zip(hip, cpu)):
        close(a, b, tol, f"{what} output {k}")
    plan = g.compile(outs, inputs, device="hip", optimize="standard").plan_summary()
    return sum(s["kind"] == "fused" and s["row_len"] > 0 for s in plan)


def _layer_norm(g, x, scale, shift, d):
    mean = g.bin("div", g.op("sum", [x], axes=[len(g.shape(x)) - 1], keepdims=True), g.scalar(float(d), "float32"))
    c = g.bin("sub", x, mean)
    var = g.bin("div", g.op("sum", [g.bin("mul", c, c)], axes=[len(g.shape(x)) - 1], keepdims=True), g.scalar(float(d), "float32"))
    y = g.bin("div", c, g.un("sqrt", g.bin("add", var, g.scalar(1e-5, "float32"))))
    return g.bin("add", g.bin("mul", y, scale), shift)


@pytest.mark.parametrize("rows,d", [(4096, 256), (300, 1024), (77, 96), (64, 1000), (5, 7)])
def test_layer_norm_forward_and_backward(rows, d):
    r = np.random.default_rng(rows + d)
    xv = r.normal(size=(rows, d)).astype(np.float32)
    sv = (1 + 0.1 * r.normal(size=d)).astype(np.float32)
    bv = (0.1 * r.normal(size=d)).astype(np.float32)
    wv = r.normal(size=(rows, d)).astype(np.float32)
    g = G()
    x, s, b, w = g.input((rows, d), "float32"), g.input((d,), "float32"), g.input((d,), "float32"), g.input((rows, d), "float32")
    y = _layer_norm(g, x, s, b, d)
    loss = g.sum_all(g.bin("mul", y, w))
    gx, gs, gb = g.grad(loss, [x, s, b])
    n = _both(g, [y, gx, gs, gb], [xv, sv, bv, wv], what=f"layernorm {rows}x{d}")
    assert n >= 2, "forward and backward should each form a row group"
    plan = g.compile([y, gx, gs, gb], [xv, sv, bv, wv], device="hip", optimize="standard").plan_summary()
    cols = sum(s.get("column_reductions", 0) for s in plan if s["kind"] == "fused")
    assert cols == 2, f"the scale and shift gradients should fold inside the backward row group: {cols}"


@pytest.mark.parametrize("shape", [(32, 8, 256), (16, 4, 96), (3, 300)])
def test_masked_softmax_forward_and_backward(shape):
    r = np.random.default_rng(1)
    L = shape[-1]
    sv = r.normal(size=shape).astype(np.float32) * 3
    mv = np.tril(np.ones((shape[-2], L), np.float32)) if len(shape) >= 2 and shape[-2] == L else (r.uniform(size=shape) > 0.2).astype(np.float32)
    wv = r.normal(size=shape).astype(np.float32)
    g = G()
    sx, m, w = g.input(shape, "float32"), g.input(mv.shape, "float32"), g.input(shape, "float32")
    masked = g.op("where", [m, g.bin("div", sx, g.scalar(np.sqrt(32.0), "float32")), g.scalar(-1e9, "float32")])
    mx = g.op("max", [masked], axes=[len(shape) - 1], keepdims=True)
    e = g.un("exp", g.bin("sub", masked, mx))
    p = g.bin("div", e, g.op("sum", [e], axes=[len(shape) - 1], keepdims=True))
    loss = g.sum_all(g.bin("mul", p, w))
    gs = g.grad(loss, [sx])[0]
    n = _both(g, [p, gs], [sv, mv, wv], what=f"softmax {shape}")
    assert n >= 2


def test_cross_entropy_on_the_python_surface():
    r = np.random.default_rng(2)
    logits = rg.tensor(r.normal(size=(512, 96)).astype(np.float32))
    labels = rg.tensor(r.integers(0, 96, size=512).astype(np.int32))
    fn = rg.value_and_grad(lambda z: nn.cross_entropy(z, labels))
    hip = rg.compile(fn, (logits,), device="hip", validate="standard")
    assert hip.report.ok, hip.report["diagnostics"]
    cpu = rg.compile(fn, (logits,), device="cpu", validate="none")
    (v1, g1), (v2, g2) = hip(logits), cpu(logits)
    close(np.array(float(v1)), np.array(float(v2)), 1e-4, "loss")
    close(g1.numpy(), g2.numpy(), 1e-4, "gradient")


def test_float64_rows():
    r = np.random.default_rng(3)
    xv = r.normal(size=(100, 300))
    g = G()
    x = g.input((100, 300))
    mx = g.op("max", [x], axes=[1], keepdims=True)
    e = g.un("exp", g.bin("sub", x, mx))
    lse = g.bin("add", g.un("log", g.op("sum", [e], axes=[1], keepdims=True)), mx)
    out = g.bin("sub", x, lse)
    gx = g.grad(g.sum_all(g.bin("mul", out, out)), [x])[0]
    assert _both(g, [out, gx], [xv], tol=1e-12, what="log-softmax f64") >= 1


@pytest.mark.parametrize("chunk", range(2))
def test_random_row_programs(chunk):
    """The row-program fuzz of the planner tests (float64 programs), on the device against the oracle."""
    r = XorShift(0x0DDBA11C0FFEE000 + chunk)
    formed = 0
    for case in range(12):
        tw = Twin()
        rows_shape = [(1,), (3,), (40,), (2, 5), (1024,)][r.below(5)]
        L = [7, 64, 96, 256, 300, 1000][r.below(6)]
        inputs = []
        for s in [rows_shape + (L,), rows_shape + (L,), rows_shape + (1,), (L,)]:
            inputs.append((0.2 + np.array([r.unit() for _ in range(int(np.prod(s)))])).reshape(s))
            tw.add_input(s, inputs[-1])
        full, per_row = _row_program(r, tw, rows_shape, L)
        outs = [tw.ids[full[-1]]] + ([tw.ids[per_row[-1]]] if per_row else [])
        y = tw.g.sum_all(outs[0])
        outs.append(tw.g.grad(y, [tw.ids[0]])[0])
        formed += _both(tw.g, outs, inputs, tol=1e-9, what=f"chunk {chunk} case {case}")
    assert formed >= 4, f"row groups formed: {formed}"
