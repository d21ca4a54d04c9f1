"""HIP kernels against the CPU oracle, op by op (the pattern of the reference's tests/metal.rs:55-178).

Bars: int32, index and byte work bit-exact; fp32 elementwise within 2 ulp of the oracle (glibc
libm vs the device math library); reductions and products within 1e-4 relative to the largest
magnitude.
"""

import numpy as np
import rustautograd_amd as rg
from rustautograd_amd import _rg
import pytest

from helpers import agree, close, op, run_graph, seq, t

pytestmark = pytest.mark.gpu

UNARY = ["neg", "exp", "log", "sqrt", "sin", "cos", "tanh", "abs", "sign", "floor"]
BINARY = ["add", "sub", "mul", "div", "pow", "maximum", "minimum", "gt", "ge"]
PATTERNS = [((4, 3), (4, 3)), ((4, 3), ()), ((), (4, 3)), ((4, 3), (3,)), ((4, 1), (1, 3)), ((2, 1, 3), (4, 1))]


@pytest.mark.parametrize("name", UNARY)
def test_unary_ops_within_two_ulp(name):
    agree(lambda g, i: op(g, name, [i[0]]), [seq((5, 7))], what=name, ulps=2)


@pytest.mark.parametrize("name", BINARY)
@pytest.mark.parametrize("shapes", PATTERNS)
def test_binary_ops_every_broadcast_pattern(name, shapes):
    a, b = shapes
    agree(lambda g, i: op(g, name, [i[0], i[1]]), [seq(a), seq(b)], what=f"{name} {a} {b}", ulps=2)


def test_where_and_fused_chains():
    agree(lambda g, i: op(g, "where", [op(g, "gt", [i[0], i[1]]), i[0], i[1]]), [seq((3, 3)), t(np.full((3, 3), 0.5))], ulps=0)

    # A chain of every fusable op in one group, over Full, Splat, Row and Broadcast inputs.
    def chain(g, i):
        x = i[0]
        y = op(g, "add", [x, i[1]])           # Row
        y = op(g, "mul", [y, i[2]])           # Splat
        y = op(g, "sub", [y, i[3]])           # Broadcast (column)
        y = op(g, "tanh", [y])
        y = op(g, "exp", [y])
        y = op(g, "log", [op(g, "add", [y, i[2]])])
        y = op(g, "div", [y, op(g, "sqrt", [op(g, "abs", [x])])])
        y = op(g, "maximum", [y, op(g, "neg", [x])])
        y = op(g, "minimum", [y, op(g, "sin", [x])])
        z = op(g, "pow", [op(g, "abs", [y]), op(g, "cos", [x])])
        w = op(g, "where", [op(g, "ge", [z, y]), z, op(g, "floor", [y])])
        return [w, op(g, "sign", [op(g, "sub", [w, x])])]
    agree(chain, [seq((64, 33)), seq((33,)), t(1.5), seq((64, 1))], what="chain", ulps=4)


def test_vectorized_and_tail_paths_of_fused_kernels():
    for n in (1, 3, 4, 1023, 1025, 4096 * 3 + 5):
        agree(lambda g, i: op(g, "mul", [op(g, "add", [i[0], i[1]]), i[0]]), [seq((n,)), seq((n,))], what=f"n={n}", ulps=0)
    agree(lambda g, i: op(g, "exp", [op(g, "mul", [i[0], i[1]])]), [seq((37, 64)), seq((64,))], what="row L%4==0", ulps=2)
    agree(lambda g, i: op(g, "exp", [op(g, "mul", [i[0], i[1]])]), [seq((37, 63)), seq((63,))], what="row L%4!=0", ulps=2)


def test_ieee_special_values():
    specials = [0.0, -0.0, 1.0, -1.0, 2.5, -2.5, np.inf, -np.inf, np.nan, 1e30, -1e30, 1e-30]
    x = t(specials)
    for name in ["exp", "log", "sqrt", "tanh", "abs", "sign", "floor", "neg"]:
        agree(lambda g, i: op(g, name, [i[0]]), [x], what=f"special {name}", ulps=2)
    trig = t([0.0, 1.0, -2.5, np.inf, -np.inf, np.nan])
    for name in ["sin", "cos"]:
        agree(lambda g, i: op(g, name, [i[0]]), [trig], what=f"special {name}", ulps=2)
    pairs = [(a, b) for a in specials for b in specials]
    a, b = t([p[0] for p in pairs]), t([p[1] for p in pairs])
    for name in ["add", "sub", "mul", "div", "maximum", "minimum", "gt", "ge"]:
        agree(lambda g, i: op(g, name, [i[0], i[1]]), [a, b], what=f"special {name}", ulps=0)
    agree(lambda g, i: op(g, "pow", [i[0], i[1]]), [t([-2.0, -2.0, -3.0, 2.0, 0.0, -2.0]), t([2.0, 3.0, -1.0, 0.5, 2.0, 0.5])],
          what="pow negative base", ulps=2)


def test_structural_ops_are_bit_exact():
    x = seq((3, 4, 5))
    agree(lambda g, i: op(g, "transpose", [i[0]], perm=[2, 0, 1]), [x], ulps=0)
    agree(lambda g, i: op(g, "broadcast_to", [i[0]], shape=[2, 3, 4, 5]), [x], ulps=0)
    agree(lambda g, i: op(g, "slice", [i[0]], starts=[1, 0, 2], stops=[3, 4, 4]), [x], ulps=0)
    agree(lambda g, i: op(g, "pad", [i[0]], starts=[1, 2, 0], shape=[5, 6, 7]), [x], ulps=0)
    for axis in range(3):
        agree(lambda g, i: op(g, "concat", [i[0], i[0], i[0]], axis=axis), [x], ulps=0)
        agree(lambda g, i: op(g, "take", [i[0], i[1]], axis=axis), [x, t([[1, 0], [2, 2]], "int32")], ulps=0)
    ix = t(np.arange(24).reshape(3, 4, 2) % 5, "int32")
    agree(lambda g, i: op(g, "take_along", [i[0], i[1]]), [x, ix], ulps=0)
    agree(lambda g, i: op(g, "take_along_grad", [i[0], i[1]], shape=[3, 4, 5]), [seq((3, 4, 2)), ix], ulps=0)
    agree(lambda g, i: op(g, "take_grad", [i[0], i[1]], axis=0, shape=[2, 5]), [seq((3, 5)), t([1, 1, 0], "int32")], ulps=0)
    agree(lambda g, i: op(g, "argmax", [i[0]]), [x])
    agree(lambda g, i: op(g, "cast", [op(g, "cast", [i[0]], dtype="int32")], dtype="float32"), [t([1.5, -1.5, 3.9])], ulps=0)
    agree(lambda g, i: op(g, "add", [i[0], i[0]]), [t([1, -2, 3], "int32")])
    agree(lambda g, i: op(g, "take", [i[0], i[1]], axis=0), [seq((3,)), t([9, -4, 1], "int32")], ulps=0)
    # Repeated and clamped indices in several rows (tests/metal.rs:317-320).
    idx = t([1, 1, 0, 4, 9, -3, 2, 2, 3, 3, 4, 0], "int32")
    agree(lambda g, i: op(g, "take_along_grad", [i[0], op(g, "reshape", [i[1]], shape=[2, 3, 2])], shape=[2, 3, 5]),
          [seq((2, 3, 2)), idx], ulps=0)


def test_casts_saturate_and_map_nan_to_zero():
    x = t([np.nan, 3e9, -3e9, 2.9, -2.9, 0.5, -0.0], "float64")
    agree(lambda g, i: op(g, "cast", [i[0]], dtype="int32"), [x])
    agree(lambda g, i: op(g, "cast", [i[0]], dtype="float32"), [t([1e300, 1.0000001, -2.5e-45], "float64")], ulps=0)


@pytest.mark.parametrize("kind", ["sum", "max", "min"])
def test_reductions_over_every_axis_set(kind):
    x = seq((3, 4, 5))
    for axes in [[0], [1], [2], [0, 2], [1, 2], [0, 1, 2], [], [0, 1]]:
        for keepdims in (True, False):
            agree(lambda g, i: op(g, kind, [i[0]], axes=axes, keepdims=keepdims), [x], tol=1e-6, what=f"{kind} {axes} {keepdims}")


@pytest.mark.parametrize("shape,axes", [((8192, 256), [1]), ((65536, 96), [1]), ((8192, 768), [0]), ((32, 256, 1024), [0, 1]),
                                        ((4, 50000), [1]), ((3 << 20,), [0]), ((2, 3000, 7), [1]), ((5, 7, 9, 11), [0, 2])])
def test_reductions_at_model_shapes(shape, axes):
    rng = np.random.default_rng(3)
    x = t(rng.normal(size=shape).astype(np.float32))
    for kind in ("sum", "max"):
        hip, cpu = run_graph("hip", lambda g, i: op(g, kind, [i[0]], axes=axes, keepdims=False), [x]), \
            run_graph("cpu", lambda g, i: op(g, kind, [i[0]], axes=axes, keepdims=False), [x])
        close(hip[0], cpu[0], 1e-4, f"{kind} {shape} {axes}")


@pytest.mark.parametrize("shape,axes", [((3, 5000, 64), [1]), ((40, 8192), [0]), ((1000, 100), [0]), ((1000, 101), [0]), ((257, 12), [0]), ((8, 4), [0])])
def test_column_reductions_repeat_exactly(shape, axes):
    """Leading-axis reductions: chunk partials folded in a fixed order by a second launch. Shapes
    cover a batch, partial column tiles, uneven chunks, a single chunk, and column counts that do
    and do not allow 16-byte loads. Three calls in a row on
    one compiled program must each match the oracle and repeat bit for bit."""
    rng = np.random.default_rng(5)
    for kind in ("sum", "max", "min"):
        g = _rg.Graph()
        i = g.input(list(shape), "float32")
        outs = [op(g, kind, [i], axes=axes, keepdims=False)]
        xs = [t(rng.normal(size=shape).astype(np.float32)) for _ in range(2)]
        hip = _rg.compile(g, outs, [xs[0]._t], "none", "hip", "none")
        cpu = _rg.compile(g, outs, [xs[0]._t], "none", "cpu", "none")
        first = None
        for x in (xs[0], xs[1], xs[0]):
            got = rg.Tensor(hip.call([x._t])[0]).numpy()
            close(got, rg.Tensor(cpu.call([x._t])[0]).numpy(), 1e-4, f"{kind} {shape} {axes}")
            if x is xs[0]:
                if first is None:
                    first = got
                else:
                    assert np.array_equal(got, first), f"{kind} {shape}: repeated call differs"


MATMUL_CASES = [((3,), (3,)), ((2, 3), (3,)), ((3,), (3, 2)), ((2, 3), (3, 4)), ((5, 2, 3), (3, 4)), ((5, 2, 3), (5, 3, 4)),
                ((2, 3), (7, 3, 4)), ((1, 2, 3), (6, 3, 4)), ((5, 1, 2, 3), (1, 4, 3, 2))]


@pytest.mark.parametrize("a,b", MATMUL_CASES)
def test_matmul_ranks_and_batches(a, b):
    agree(lambda g, i: op(g, "matmul", [i[0], i[1]]), [seq(a), seq(b)], tol=2e-6, what=f"matmul {a} {b}")


def _swap(g, x, rank):
    p = list(range(rank))
    p[-2], p[-1] = p[-1], p[-2]
    return op(g, "transpose", [x], perm=p)


@pytest.mark.parametrize("m,k,n", [(256, 256, 768), (300, 70, 130), (8192, 256, 96), (256, 8192, 768), (64, 64, 64), (33, 17, 65),
                                   (8192, 1024, 256), (1024, 8192, 256), (8200, 260, 264), (33, 4096, 65),
                                   (4096, 512, 128), (128, 4096, 384)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_mfma_products_with_transpose_flags(m, k, n, ta, tb):
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a = rng.normal(size=(k, m) if ta else (m, k)).astype(np.float32)
    b = rng.normal(size=(n, k) if tb else (k, n)).astype(np.float32)

    def build(g, i):
        x = _swap(g, i[0], 2) if ta else i[0]
        y = _swap(g, i[1], 2) if tb else i[1]
        return op(g, "matmul", [x, y])
    hip = run_graph("hip", build, [t(a), t(b)], optimize="standard")[0]
    want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    close(hip, want, 1e-4, f"gemm {m}x{k}x{n} ta={ta} tb={tb}")


@pytest.mark.parametrize("m,k,n,ta", [(8192, 256, 768, False), (256, 8192, 768, True), (1024, 8192, 256, True), (33, 17, 65, False),
                                      (3, 5, 7, False), (300, 70, 132, True)])
def test_products_with_a_bias_operand(m, k, n, ta):
    """A bias add folded into the product before it: added in the MFMA kernel's epilogue, after
    the split-K sum for split products, or by a separate pass for products off the matrix cores."""
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    a = rng.normal(size=(k, m) if ta else (m, k)).astype(np.float32)
    w = rng.normal(size=(k, n)).astype(np.float32)
    b = rng.normal(size=(n,)).astype(np.float32)

    def build(g, i):
        x = _swap(g, i[0], 2) if ta else i[0]
        return op(g, "add", [op(g, "matmul", [x, i[1]]), op(g, "broadcast_to", [i[2]], shape=[m, n])])
    hip = run_graph("hip", build, [t(a), t(w), t(b)], optimize="standard")[0]
    want = (a.T if ta else a).astype(np.float64) @ w.astype(np.float64) + b.astype(np.float64)
    close(hip, want, 1e-4, f"biased product {m}x{k}x{n} ta={ta}")


def test_split_products_feed_later_steps():
    """K-split products whose partial sums are folded later, just before the first step that
    reads the product: an elementwise group, another product and a program output."""
    rng = np.random.default_rng(11)
    a = rng.normal(size=(8192, 256)).astype(np.float32)
    b = rng.normal(size=(8192, 768)).astype(np.float32)
    c = rng.normal(size=(768, 64)).astype(np.float32)

    def build(g, i):
        y = op(g, "matmul", [_swap(g, i[0], 2), i[1]])
        z = op(g, "mul", [y, y])
        return [z, op(g, "matmul", [y, i[2]]), y]
    hip = run_graph("hip", build, [t(a), t(b), t(c)], optimize="standard")
    y = a.T.astype(np.float64) @ b.astype(np.float64)
    close(hip[0], y * y, 2e-4, "square of a split product")
    close(hip[1], y @ c.astype(np.float64), 1e-4, "product of a split product")
    close(hip[2], y, 1e-4, "split product")


@pytest.mark.parametrize("a,b", [((5, 1, 96, 64), (1, 4, 64, 96)), ((3, 67, 129), (3, 129, 65)), ((2, 3, 128, 64), (3, 64, 256))])
def test_batched_products_with_broadcast_and_odd_strides(a, b):
    """Per-batch offset tables (broadcast batches) and batch strides that are not multiples of 4."""
    rng = np.random.default_rng(sum(a) + sum(b))
    x, y = rng.normal(size=a).astype(np.float32), rng.normal(size=b).astype(np.float32)
    hip = run_graph("hip", lambda g, i: op(g, "matmul", [i[0], i[1]]), [t(x), t(y)], optimize="standard")[0]
    close(hip, x.astype(np.float64) @ y.astype(np.float64), 1e-4, f"matmul {a} {b}")


def test_batched_attention_products():
    rng = np.random.default_rng(5)
    q = rng.normal(size=(4, 8, 256, 32)).astype(np.float32)
    kk = rng.normal(size=(4, 8, 256, 32)).astype(np.float32)

    def build(g, i):
        s = op(g, "matmul", [i[0], _swap(g, i[1], 4)])
        return [s, op(g, "matmul", [s, i[1]])]
    hip = run_graph("hip", build, [t(q), t(kk)], optimize="standard")
    s = q.astype(np.float64) @ np.swapaxes(kk, -1, -2).astype(np.float64)
    close(hip[0], s, 1e-5, "qk")
    close(hip[1], s @ kk.astype(np.float64), 1e-5, "sv")


def test_random_bits_are_identical_to_cpu():
    key = t([7, -11], "int32")

    def build(g, i):
        return [op(g, "random_uniform", [i[0]], shape=[1000], dtype="float32"), op(g, "key_split", [i[0]], n=5),
                op(g, "random_uniform", [i[0]], shape=[10], dtype="float64"), op(g, "random_uniform", [i[0]], shape=[1 << 16], dtype="float32")]
    hip = run_graph("hip", build, [key])
    cpu = run_graph("cpu", build, [key])
    for a, b in zip(hip, cpu):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_normal_sampling_matches_cpu():
    key = t([3, 4], "int32")
    agree(lambda g, i: op(g, "random_normal", [i[0]], shape=[4096], dtype="float32"), [key], ulps=1)
    agree(lambda g, i: op(g, "random_normal", [i[0]], shape=[512], dtype="float64"), [key], ulps=4)


def test_sort_and_scan_kernels():
    x = t([[3.0, 1.0, 3.0, np.nan, 2.0, -1.0, 3.0, 0.5]] * 3)
    agree(lambda g, i: op(g, "arg_top_k", [i[0]], k=3), [x])
    agree(lambda g, i: op(g, "arg_top_k", [i[0]], k=8), [x])
    agree(lambda g, i: op(g, "cumsum", [i[0]], reverse=True), [seq((3, 8))], ulps=0)
    agree(lambda g, i: op(g, "cumsum", [i[0]], reverse=False), [t(np.arange(12).reshape(3, 4), "int32")])


@pytest.mark.parametrize("rows,v,k,dtype", [(1, 96, 96, "float32"), (70, 96, 20, "float32"), (5, 300, 300, "float32"),
                                            (3, 4096, 7, "float64"), (2, 5000, 5, "float32"), (4096, 4096, 1, "float32")])
def test_top_k_and_argsort_rank_rows_like_the_oracle(rows, v, k, dtype):
    """Rows up to 4096 long rank every position in one block; longer rows, and many long rows
    with a small k, choose positions in turn. Ties (a coarse grid of values), NaNs and both ends
    of k must give the oracle's order."""
    rng = np.random.default_rng(rows * 31 + v + k)
    x = np.round(rng.normal(size=(rows, v)) * 4) / 4
    x[rng.random(size=(rows, v)) < 0.02] = np.nan
    agree(lambda g, i: op(g, "arg_top_k", [i[0]], k=k), [t(x.astype(dtype), dtype)])


def test_float64_programs_run_on_the_device():
    def build(g, i):
        e = op(g, "exp", [i[0]])
        w = op(g, "cast", [e], dtype="float64")
        l = op(g, "log", [w])
        back = op(g, "cast", [l], dtype="float32")
        return [op(g, "mul", [back, i[0]]), l]
    agree(build, [seq((4,))], tol=2e-6)


def test_vectorized_structural_paths():
    x = seq((4, 8, 16, 32))
    agree(lambda g, i: op(g, "transpose", [i[0]], perm=[0, 2, 1, 3]), [x], ulps=0)
    agree(lambda g, i: op(g, "transpose", [op(g, "reshape", [i[0]], shape=[4, 16, 2, 4, 32])], perm=[2, 0, 3, 1, 4]), [x], ulps=0)
    agree(lambda g, i: op(g, "broadcast_to", [i[0]], shape=[3, 4, 8, 16, 32]), [x], ulps=0)
    agree(lambda g, i: op(g, "broadcast_to", [i[0]], shape=[4, 8, 16, 32]), [t(-1e9)], ulps=0)
    agree(lambda g, i: op(g, "broadcast_to", [i[0]], shape=[4, 8, 16, 32]), [seq((16, 1))], ulps=0)
    agree(lambda g, i: op(g, "slice", [i[0]], starts=[1, 0, 4, 0], stops=[3, 8, 12, 32]), [x], ulps=0)
    agree(lambda g, i: op(g, "slice", [i[0]], starts=[0, 0, 0, 1], stops=[4, 8, 16, 29]), [x], ulps=0)


def test_scatter_add_at_embedding_shapes_is_bit_exact():
    rng = np.random.default_rng(11)
    ct = t(rng.normal(size=(32, 256, 256)).astype(np.float32))
    idx = t(rng.integers(0, 96, size=(32, 256)), "int32")
    agree(lambda g, i: op(g, "take_grad", [i[0], i[1]], axis=0, shape=[96, 256]), [ct, idx], ulps=0)
    # Index chunks beyond the LDS list, a middle axis, and clamped entries.
    ct2 = t(rng.normal(size=(3, 9000, 5)).astype(np.float32))
    idx2 = t(rng.integers(-3, 12, size=(9000,)), "int32")
    agree(lambda g, i: op(g, "take_grad", [i[0], i[1]], axis=1, shape=[3, 10, 5]), [ct2, idx2], ulps=0)
    # One row hit by every entry (long in-order sums across two chunks), in float64 and float32.
    for dtype in ("float64", "float32"):
        ct3 = t(rng.normal(size=(10001, 3)), dtype)
        idx3 = t(np.where(np.arange(10001) % 97 == 0, 2, 7), "int32")
        agree(lambda g, i: op(g, "take_grad", [i[0], i[1]], axis=0, shape=[9, 3]), [ct3, idx3], ulps=0)


I32_MIN, I32_MAX = -2 ** 31, 2 ** 31 - 1
INT_PAIRS = [(I32_MAX, 1), (I32_MIN, -1), (65536, 65536), (46341, 46341), (I32_MIN, I32_MIN), (I32_MAX, I32_MAX),
             (I32_MIN, 1), (-1, I32_MIN), (0, I32_MIN), (123456789, -987654321), (-7, 3), (I32_MAX, I32_MIN)]


def _wrap32(v):
    v &= 0xFFFFFFFF
    return v - 2 ** 32 if v >= 2 ** 31 else v


INT_RULES = {"add": lambda a, b: _wrap32(a + b), "sub": lambda a, b: _wrap32(a - b), "mul": lambda a, b: _wrap32(a * b),
             "gt": lambda a, b: int(a > b), "ge": lambda a, b: int(a >= b)}


@pytest.mark.parametrize("name", sorted(INT_RULES))
def test_int32_ops_wrap_and_compare_bit_exactly(name):
    """int32 add/sub/mul wrap modulo 2^32 and comparisons hold at the bounds (src/plan.rs:1272-1287),
    in every broadcast mode; checked against the oracle and against the closed form."""
    a = t([p[0] for p in INT_PAIRS], "int32")
    b = t([p[1] for p in INT_PAIRS], "int32")
    hip, _ = agree(lambda g, i: op(g, name, [i[0], i[1]]), [a, b], what=name)
    assert hip[0].tolist() == [INT_RULES[name](x, y) for x, y in INT_PAIRS]
    s = t(I32_MAX, "int32")
    hip, _ = agree(lambda g, i: op(g, name, [i[0], i[1]]), [s, b], what=f"{name} scalar lhs")
    assert hip[0].tolist() == [INT_RULES[name](I32_MAX, y) for _, y in INT_PAIRS]
    hip, _ = agree(lambda g, i: op(g, name, [i[0], i[1]]), [a, s], what=f"{name} scalar rhs")
    assert hip[0].tolist() == [INT_RULES[name](x, I32_MAX) for x, _ in INT_PAIRS]
    col = t(np.array([p[0] for p in INT_PAIRS], dtype=np.int32).reshape(12, 1), "int32")
    row = t(np.array([p[1] for p in INT_PAIRS], dtype=np.int32).reshape(1, 12), "int32")
    hip, _ = agree(lambda g, i: op(g, name, [i[0], i[1]]), [col, row], what=f"{name} general broadcast")
    assert hip[0].tolist() == [[INT_RULES[name](x, y) for _, y in INT_PAIRS] for x, _ in INT_PAIRS]


def _sweep(lo, hi, n, seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([np.linspace(lo, hi, n // 2), rng.uniform(lo, hi, n - n // 2)]).astype(np.float32)


WIDE = {
    "exp": np.concatenate([_sweep(-104.0, 89.0, 4096, 1), np.float32([-87.33655, 88.72283, 88.72284, -103.97208])]),
    "log": np.concatenate([_sweep(1e-6, 1e6, 4096, 2), np.float32([1e-45, 1e-40, 1.17549435e-38, 3.4028235e38])]),
    "sin": np.concatenate([_sweep(-1e4, 1e4, 4096, 3), np.float32([1e5, -1e6, 1e-30, 3.1415927])]),
    "cos": np.concatenate([_sweep(-1e4, 1e4, 4096, 4), np.float32([1e5, -1e6, 1e-30, 1.5707964])]),
    "tanh": np.concatenate([_sweep(-12.0, 12.0, 4096, 5), np.float32([-10.0, 10.0, 9.01, -9.01, 1e-20])]),
    "sqrt": np.concatenate([_sweep(0.0, 1e30, 4096, 6), np.float32([1e-45, 1e-40, 3.4028235e38])]),
}


@pytest.mark.parametrize("name", sorted(WIDE))
def test_fp32_unary_ops_over_wide_ranges_within_two_ulp(name):
    """Near overflow and underflow of exp, large arguments of sin and cos, saturation of tanh, the
    subnormal and huge ends of log and sqrt: the device's math stays within 2 ulp of glibc."""
    agree(lambda g, i: op(g, name, [i[0]]), [t(WIDE[name])], what=f"wide {name}", ulps=2)
    # The same values through a fused group (the JIT path) rather than the single-op kernel.
    agree(lambda g, i: op(g, "add", [op(g, name, [i[0]]), i[1]]), [t(WIDE[name]), t(0.0)], what=f"wide fused {name}", ulps=2)


def test_fp32_pow_over_wide_ranges_within_two_ulp():
    rng = np.random.default_rng(7)
    base = np.concatenate([rng.uniform(0.0, 4.0, 3000), rng.uniform(-3.0, 0.0, 500).round(), np.float32([2.0, 10.0, 0.5, 1.0001])])
    expo = np.concatenate([rng.uniform(-40.0, 40.0, 3000), rng.integers(-9, 10, 500).astype(np.float64), np.float32([127.0, 38.0, 149.0, 80000.0])])
    agree(lambda g, i: op(g, "pow", [i[0], i[1]]), [t(base.astype(np.float32)), t(expo.astype(np.float32))], what="wide pow", ulps=2)


def _product_graph(sa, sb, ta, tb):
    """op(A) @ op(B) with the transposes written as nodes, which the optimizer turns into flags."""
    def build(g, i):
        a = op(g, "transpose", [i[0]], perm=[1, 0]) if ta else i[0]
        b = op(g, "transpose", [i[1]], perm=[1, 0]) if tb else i[1]
        return op(g, "matmul", [a, b])
    return build


# (m, k, n, ta, tb): products with few rows and a long K (row-major or transposed right operand)
# and outer products with a short K, which the HIP backend streams through its skinny kernels.
SKINNY = [
    (8, 4096, 4096, False, False), (1, 512, 256, False, False), (16, 2048, 1024, True, False), (9, 777, 68, False, False),
    (8, 4096, 4096, False, True), (5, 1024, 100, False, True), (16, 512, 640, False, True),
    (4096, 8, 1024, True, False), (2048, 1, 1024, False, False), (1024, 16, 1024, False, True), (1024, 3, 2048, True, True),
    (8, 8, 4096, False, True),
    # matrix-vector products (run as their transposes) and tiny outputs with a long K
    (4096, 2048, 1, False, False), (2048, 4096, 1, True, False), (1000, 1000, 1, True, True), (1001, 512, 1, True, False),
    (8, 4096, 8, False, False), (3, 2000, 5, True, True), (16, 600, 16, False, True),
    (4, 3000, 4, True, False), (2, 9000, 3, False, False), (16, 512, 20, False, True), (128, 512, 128, False, True),
    # a tied embedding's gradient (C3's head): MFMA tiles, not the tiny-output kernel
    (96, 4096, 128, True, False),
]


@pytest.mark.parametrize("m,k,n,ta,tb", SKINNY)
def test_skinny_products_match_numpy_and_the_oracle(m, k, n, ta, tb):
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.normal(size=(k, m) if ta else (m, k)).astype(np.float32)
    b = rng.normal(size=(n, k) if tb else (k, n)).astype(np.float32)
    build = _product_graph(a.shape, b.shape, ta, tb)
    hip = run_graph("hip", build, [t(a), t(b)], optimize="standard")[0]
    want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    scale = np.abs(want).max()
    assert np.abs(hip - want).max() <= 1e-4 * scale, f"{np.abs(hip - want).max() / scale:.2e} relative to max|want|"
    if m * k * n <= (1 << 27):
        cpu = run_graph("cpu", build, [t(a), t(b)], optimize="standard")[0]
        close(hip, cpu, 1e-4, "skinny vs oracle")


# Independent streamed products of one program: rows and dot kernels (8 rows), outer products of
# each operand layout and K of 8 and 4, and tiny outputs over K whose single kernel has 4, 8 and 16
# waves.
GROUPED_STREAMED = [
    (8, 4096, 2048, False, False), (8, 4096, 1024, False, True), (2048, 8, 1024, True, False), (1024, 4, 2048, False, False),
    (8, 2048, 8, False, False), (4, 8000, 4, True, False), (1024, 8, 1024, False, True), (8, 4096, 8, False, True),
]


def test_streamed_products_launched_together_match_single_launches(monkeypatch):
    """Adjacent independent streamed products run as one launch of k_stream_group, each block
    running its own product's block code: the outputs equal the single launches' (RG_HIP_PAIR=0)
    bit for bit, and numpy's float64 products within 1e-4 of the largest value."""
    rng = np.random.default_rng(11)
    ops = []
    for m, k, n, ta, tb in GROUPED_STREAMED:
        ops.append(rng.normal(size=(k, m) if ta else (m, k)).astype(np.float32))
        ops.append(rng.normal(size=(n, k) if tb else (k, n)).astype(np.float32))

    def build(g, i):
        return [_product_graph(None, None, ta, tb)(g, i[2 * q:2 * q + 2]) for q, (m, k, n, ta, tb) in enumerate(GROUPED_STREAMED)]

    def compiled():
        g = _rg.Graph()
        ids = [g.input(list(x.shape), "float32") for x in ops]
        return _rg.compile(g, build(g, ids), [t(x)._t for x in ops], "none", "hip", "standard")

    monkeypatch.setenv("RG_HIP_PAIR", "0")
    single = compiled()
    monkeypatch.delenv("RG_HIP_PAIR")
    grouped = compiled()
    moved = [k for k, r in enumerate(grouped.step_runs_in()) if r != k]
    assert all(r == k for k, r in enumerate(single.step_runs_in())) and len(moved) >= 3, grouped.step_runs_in()
    out0 = [rg.Tensor(r).numpy() for r in single.call([t(x)._t for x in ops])]
    out1 = [rg.Tensor(r).numpy() for r in grouped.call([t(x)._t for x in ops])]
    for q, (m, k, n, ta, tb) in enumerate(GROUPED_STREAMED):
        a, b = ops[2 * q], ops[2 * q + 1]
        want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
        assert np.array_equal(out0[q].view(np.uint32), out1[q].view(np.uint32)), (m, k, n, ta, tb)
        assert np.abs(out1[q] - want).max() <= 1e-4 * np.abs(want).max(), (m, k, n, ta, tb)
