"""Random graphs and their gradients on the HIP device against the CPU oracle.

The intent of the reference's tests/metal.rs:193-247 (`random_graphs_agree_with_cpu`): random
elementwise, broadcast, reduction, product and select graphs, with the gradient of their last
value, planned for the device and run there, then compared with the oracle's CPU plan of the same
graph. The generated-kernel paths meet random inputs this way: broadcast strides baked into fused
kernels (magic-number division), the float4 vector body and its scalar tail, merged launches of
small groups, row groups with their row and column reductions, aliasing outputs, the streaming and
matrix-core products.

Shapes cross the vector width (multiples of 4 and not), the block size (up to 1030 x 1024) and
the broadcast forms (scalars, rows, columns, (1, n) and (n, 1)). Several hundred cases run in
fixed-seed chunks; the first failing case stops its chunk with its seed, case and output named.

Tolerance, condition-aware: random graphs cancel (a value normalized by its own sum has a
gradient that is a small difference of large terms), so a fixed relative bound is either loose
or fails on correct float32 arithmetic. Each float32 case is therefore also evaluated in float64
on the oracle (the same graph over the same inputs), and the device's largest error against it
must be within 8 times the oracle's own float32 error plus 1e-6 of the largest magnitude (the
device may sum in another order, not be less accurate), or within FLOOR of max(1, largest
magnitude). The floor is for outputs so ill-conditioned that one ulp of an intermediate shows:
sin of a full sum of 10280 values near 7200 turns the sum's last bit (4.9e-4) into an output
error of 3.3e-4, and the oracle's single float32 evaluation may happen to land closer. FLOOR is
a tenth of the reference's bound. NaN and infinity positions must equal the oracle's float32
ones. Float64 cases (a fifth; the double2 paths) compare with the oracle at
1e-9 of the largest magnitude plus 1e-12 absolute: inputs lie in [0.2, 1.2), and an output that
cancels to rounding noise (a gradient of 1e-31 on one side, -0.0 on the other) has no relative
accuracy to compare. The reference compares at 5e-3 of max(1, max|cpu|) (tests/metal.rs:33-40,
243).

`DEVICE` is the device under test; tests/test_fuzz_checks.py runs the same generator against the
device-flavoured plan on the oracle, on the CPU.
"""

import numpy as np
import pytest

from helpers import G

pytestmark = pytest.mark.gpu

DEVICE = "hip"
FLOOR = 5e-4


class Rng:
    """xorshift64 (the reference tests' generator, tests/engine.rs:18-32)."""

    def __init__(self, seed):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self):
        s = self.s
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        self.s = s
        return s

    def below(self, n):
        return self.next() % n

    def values(self, n):
        return 0.2 + (np.array([self.next() % 1000 for _ in range(n)], np.float64) / 1000.0)


class Builder:
    """A random graph under construction: `pool` holds the ids of the values made so far."""

    def __init__(self, r, dtype):
        self.r, self.dtype, self.g = r, dtype, G()
        self.pool, self.inputs = [], []

    def input(self, shape):
        self.inputs.append(self.r.values(int(np.prod(shape)) if shape else 1).reshape(shape).astype(self.dtype))
        self.pool.append(self.g.input(shape, self.dtype))

    def scalar(self, v):
        return self.g.scalar(v, self.dtype)

    def shape(self, x):
        return self.g.shape(x)

    def add(self, make):
        try:
            self.pool.append(make())
        except Exception as e:  # shapes that do not combine are skipped, as the reference's `if let Ok`
            if type(e).__name__ != "DiagnosticError":
                raise

    def step(self, op_id):
        g, r = self.g, self.r
        x = self.pool[len(self.pool) - 1 - r.below(min(len(self.pool), 4))]
        y = self.pool[r.below(len(self.pool))]
        binary = ["add", "sub", "mul", "div", "maximum", "minimum"]
        if op_id < 6:
            return self.add(lambda: g.bin(binary[op_id], x, y))
        if op_id < 11:
            unary = ["tanh", "abs", "sin", "neg", "cos"][op_id - 6]
            return self.add(lambda: g.un(unary, x))
        if op_id == 11:  # bounded exponential, and sqrt / log of positive values
            return self.add(lambda: g.un("exp", g.un("tanh", x)))
        if op_id == 12:
            return self.add(lambda: g.un("sqrt", g.bin("add", g.un("abs", x), self.scalar(0.25))))
        if op_id == 13:
            return self.add(lambda: g.un("log", g.bin("add", g.un("abs", x), self.scalar(0.5))))
        if op_id == 14:
            n = int(np.prod(self.shape(x))) if self.shape(x) else 1
            return self.add(lambda: g.un("reshape", x, shape=[n]))
        if op_id == 15:
            perm = list(range(len(self.shape(x))))[::-1]
            return self.add(lambda: g.un("transpose", x, perm=perm))
        if op_id == 16:
            axes = [d for d in range(len(self.shape(x))) if r.next() % 2 == 0]
            kind = ["sum", "sum", "max", "min"][r.below(4)]
            return self.add(lambda: g.op(kind, [x], axes=axes, keepdims=r.next() % 2 == 0))
        if op_id == 17:
            return self.add(lambda: g.bin("matmul", x, y))
        if op_id == 18:
            return self.add(lambda: g.op("where", [g.bin("gt", x, y), x, y]))
        if op_id == 19:
            v = [0.5, 1.0, 2.0, -1.5][r.below(4)]
            return self.add(lambda: g.bin(["add", "mul"][r.below(2)], x, self.scalar(v)))
        if op_id == 20:  # a last-axis reduction broadcast back: the row-group pattern
            sx = self.shape(x)
            if not sx:
                return None
            kind = ["sum", "max"][r.below(2)]
            return self.add(lambda: g.bin(["sub", "div"][r.below(2)], x,
                                          g.bin("add", g.op(kind, [x], axes=[len(sx) - 1], keepdims=True), self.scalar(1.5))))
        if op_id == 21:
            return self.add(lambda: g.un("stop_gradient", x))
        raise AssertionError(op_id)


SIZES_A = [1, 3, 8, 40, 300, 1030]
SIZES_B = [1, 7, 64, 257, 600, 1024]


def random_case(r, dtype):
    """One random program: (graph, outputs, inputs); outputs are two values, the last value's sum
    and its gradient with respect to the first input. The structure depends only on `r`, not on
    `dtype`."""
    b = Builder(r, dtype)
    da, db = SIZES_A[r.below(len(SIZES_A))], SIZES_B[r.below(len(SIZES_B))]
    pool = [(), (db,), (da, db), (1, db), (da, 1)]
    for s in [(da, db), pool[r.below(5)], pool[r.below(5)]]:
        b.input(s)
    for _ in range(2 + r.below(20)):
        b.step(r.below(22))
    last = b.pool[-1]
    y = b.g.sum_all(last)
    outs = [b.pool[r.below(len(b.pool))] for _ in range(2)] + [y] + b.g.grad(y, [b.pool[0]])
    return b.g, outs, b.inputs


def check_case(g, outs, inputs, what, device=DEVICE, exact=None):
    """The device's outputs against the oracle's. `exact` is (graph, outputs) of the same program
    in float64, for float32 cases."""
    got = g.eval(outs, inputs, device=device, optimize="standard")
    want = g.eval(outs, inputs, device="cpu", optimize="none")
    truth = exact[0].eval(exact[1], [x.astype(np.float64) for x in inputs], device="cpu", optimize="none") if exact else want
    for k, (u, v, t) in enumerate(zip(got, want, truth)):
        assert u.shape == v.shape, f"{what} output {k}: shape {u.shape} vs {v.shape}"
        for name, mask in (("NaN", np.isnan), ("+inf", lambda a: np.isposinf(a)), ("-inf", lambda a: np.isneginf(a))):
            assert np.array_equal(mask(u), mask(v)), f"{what} output {k}: {name} positions differ"
        fin = np.isfinite(u) & np.isfinite(v) & np.isfinite(t)
        u, v, t = (np.where(fin, a, 0.0).astype(np.float64) for a in (u, v, t))
        scale = float(np.abs(t).max())
        if exact is None:
            bad = np.abs(u - v) > 1e-9 * scale + 1e-12
            assert not bad.any(), f"{what} output {k}[{int(np.argmax(bad))}]: {u.ravel()[np.argmax(bad)]!r} vs {v.ravel()[np.argmax(bad)]!r}"
            continue
        e_dev, e_cpu = float(np.abs(u - t).max()), float(np.abs(v - t).max())
        assert e_dev <= max(8.0 * e_cpu + 1e-6 * scale, FLOOR * max(1.0, scale)), \
            f"{what} output {k}: error against float64 {e_dev:.3e}, the oracle's float32 error {e_cpu:.3e}, magnitude {scale:.3e}"


def run_chunk(seed, cases, device=DEVICE):
    r = Rng(seed)
    for case in range(cases):
        dtype = "float64" if r.below(5) == 0 else "float32"
        at = r.s
        g, outs, inputs = random_case(r, dtype)
        exact = None
        if dtype == "float32":
            twin = Rng(0)
            twin.s = at
            g64, outs64, _ = random_case(twin, "float64")
            exact = (g64, outs64)
        check_case(g, outs, inputs, f"seed {seed:#x} case {case} ({dtype})", device, exact)


@pytest.mark.parametrize("chunk", range(8))
def test_random_graphs_on_the_device_agree_with_the_oracle(chunk):
    seed = 0xFEEDFACECAFEBEEF + chunk
    print(f"device fuzz chunk {chunk}, seed {seed:#x}, 50 cases", flush=True)
    run_chunk(seed, 50)
