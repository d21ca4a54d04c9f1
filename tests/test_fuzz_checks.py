"""The device fuzz of tests/test_hip_fuzz.py, checked on the CPU: the same generator and
comparison against the device-flavoured plan on the oracle (`cpu_devplan`: device fusion, row
groups, split sums, level order), and the comparison must fail on a planted difference."""

import numpy as np
import pytest

from conftest import DEVPLAN
from test_hip_fuzz import Rng, check_case, random_case, run_chunk


@pytest.mark.parametrize("chunk", range(2))
def test_fuzz_generator_agrees_on_the_device_plan(chunk):
    run_chunk(0xFEEDFACECAFEBEEF + chunk, 25, device=DEVPLAN)


def test_fuzz_generator_reaches_the_kernel_paths():
    """Across the first chunk: fused groups, row groups, products, broadcasts and float64 cases."""
    r = Rng(0xFEEDFACECAFEBEEF)
    kinds, f64, rows = set(), 0, 0
    for case in range(50):
        dtype = "float64" if r.below(5) == 0 else "float32"
        g, outs, inputs = random_case(r, dtype)
        f64 += dtype == "float64"
        plan = g.compile(outs, inputs, device=DEVPLAN, optimize="standard").plan_summary()
        kinds |= {s["kind"] for s in plan}
        kinds |= {s.get("op") for s in plan if s["kind"] == "instr"}
        rows += sum(s["kind"] == "fused" and s["row_len"] > 0 for s in plan)
    assert {"fused", "instr"} <= kinds and rows >= 5 and f64 >= 5, (kinds, rows, f64)
    assert any(k in kinds for k in ("matmul", "matmul_t")), kinds


def test_fuzz_comparison_catches_a_planted_difference():
    """A result 1 % off everywhere fails the float64-referenced comparison."""
    from helpers import G

    def graph(dtype, factor):
        g = G()
        x = g.input((40, 257), dtype)
        y = g.bin("mul", g.un("tanh", x), g.scalar(factor, dtype))
        return g, [y]
    inputs = [np.linspace(0.2, 1.2, 40 * 257).reshape(40, 257).astype(np.float32)]
    g, outs = graph("float32", 1.0)
    exact = graph("float64", 1.0)
    check_case(g, outs, inputs, "same", device=DEVPLAN, exact=exact)
    planted, planted_outs = graph("float32", 1.01)

    class Mixed:
        """The planted graph as the device under test, the true one as the oracle."""
        def eval(self, outs, inputs, device, optimize):
            return planted.eval(planted_outs, inputs, device, optimize) if device == DEVPLAN else g.eval(outs, inputs, device, optimize)
    with pytest.raises(AssertionError):
        check_case(Mixed(), outs, inputs, "planted", device=DEVPLAN, exact=exact)


def test_split_full_sum_with_keepdims_keeps_the_rank():
    """Found by the device fuzz: the device rewrite of a large full sum (last axis first, then the
    rest) kept `keepdims` only on its second half, so sum(x, all axes, keepdims) of a matrix came
    out with one dimension instead of two and a full sum of it failed to compile. Device and CPU
    plans now agree on shapes and values."""
    from helpers import G
    g = G()
    x = g.input((1024, 300), "float32")
    s = g.op("sum", [x], axes=[0, 1], keepdims=True)
    total = g.sum_all(s)
    y = g.bin("sub", x, s)
    inputs = [np.linspace(-1.0, 1.2, 1024 * 300).reshape(1024, 300).astype(np.float32)]
    dev = g.eval([s, total, y], inputs, device=DEVPLAN, optimize="standard")
    cpu = g.eval([s, total, y], inputs, device="cpu", optimize="none")
    assert [a.shape for a in dev] == [a.shape for a in cpu] == [(1, 1), (), (1024, 300)]


def test_row_group_reducing_a_row_level_value_compiles_for_gfx950():
    """Found by the device fuzz (chunk 5, case 9): a row group whose reduction reads a row-level
    value (here the negated constant upstream gradient of `x - max(x)`, summed over the row) was
    generated as if the value held a whole row, and its kernel did not compile. The generator now
    reduces the value over the row's positions; the kernels compile for gfx950 (no device needed)
    and the device-flavoured plan agrees with the CPU plan."""
    from rustautograd_amd import _rg
    from test_abi import _compile_check
    r = Rng(0xFEEDFACECAFEBEEF + 5)
    for case in range(10):
        dtype = "float64" if r.below(5) == 0 else "float32"
        g, outs, inputs = random_case(r, dtype)
    plan = g.compile(outs, inputs, device=DEVPLAN, optimize="standard").plan_summary()
    assert any(s["kind"] == "fused" and s["row_len"] > 0 and s["input_kinds"] == ["splat"] for s in plan), plan
    words, _ = _rg.plan_words(g.g, list(outs), "hip", "standard")
    n, err = _compile_check(list(words))
    assert n >= 1, err
    check_case(g, outs, inputs, "chunk 5 case 9", device=DEVPLAN)
