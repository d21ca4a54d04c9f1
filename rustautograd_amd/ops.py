"""The functional API: elementwise math, selection, shape manipulation, sorting and the
constructors of constant tensors. Each function is one or a few engine operations (see
`tensor.apply`); names and argument conventions are those of the reference's python/rg/_core.py.
"""

import numpy as np

from .tensor import Tensor, Tracer, Value, apply, error, filled, first_dtype, tensor, _from_array


def _normalize_axis(x, axis):
    return axis if axis >= 0 else x.ndim + axis


def _as_index(idx):
    return idx if isinstance(idx, (Tensor, Tracer)) else tensor(idx)


# ---- elementwise ----

def _unary(op):
    def fn(x):
        return apply(op, x)
    fn.__name__ = op
    fn.__doc__ = f"Elementwise `{op}`."
    return fn


exp = _unary("exp")
log = _unary("log")
sqrt = _unary("sqrt")
sin = _unary("sin")
cos = _unary("cos")
tanh = _unary("tanh")
floor = _unary("floor")
abs = _unary("abs")
sign = _unary("sign")
stop_gradient = _unary("stop_gradient")


def maximum(a, b):
    """Elementwise maximum; NaN wins over any number."""
    return apply("maximum", a, b)


def minimum(a, b):
    """Elementwise minimum; NaN wins over any number."""
    return apply("minimum", a, b)


def square(x):
    return x * x


def clip(x, low, high):
    return minimum(maximum(x, low), high)


def equal(a, b):
    """1 where a == b (as a >= b and b >= a, in the operands' dtype), else 0."""
    return apply("ge", a, b) * apply("ge", b, a)


def not_equal(a, b):
    return 1 - equal(a, b)


def where(c, a, b):
    """`a` where `c` is nonzero, else `b`, elementwise with broadcasting. A condition of another
    dtype is cast to the branches' dtype first."""
    branch_dtype = first_dtype((a, b))
    if branch_dtype is not None and isinstance(c, Value) and c.dtype != branch_dtype:
        c = c.cast(branch_dtype)
    return apply("where", c, a, b)


def matmul(a, b):
    return apply("matmul", a, b)


# ---- shape ----

def reshape(x, *shape):
    return x.reshape(*shape)


def transpose(x, *perm):
    return x.transpose(*perm)


def broadcast_to(x, shape):
    return apply("broadcast_to", x, shape=list(shape))


def swapaxes(x, a, b):
    order = list(range(x.ndim))
    a, b = _normalize_axis(x, a), _normalize_axis(x, b)
    order[a], order[b] = order[b], order[a]
    return x.transpose(order)


def expand_dims(x, axis):
    at = axis + x.ndim + 1 if axis < 0 else axis
    return x.reshape(tuple(x.shape[:at]) + (1,) + tuple(x.shape[at:]))


def squeeze(x, axis=None):
    if axis is None:
        drop = {i for i, d in enumerate(x.shape) if d == 1}
    else:
        drop = {_normalize_axis(x, a) for a in (axis if isinstance(axis, (tuple, list)) else (axis,))}
    longer = [a for a in drop if x.shape[a] != 1]
    if longer:
        raise error("SHAPE_MISMATCH", {"shape": x.shape, "axes": sorted(drop)}, "squeeze_of_axis_longer_than_one")
    return x.reshape([n for a, n in enumerate(x.shape) if a not in drop])


def concatenate(xs, axis=0):
    parts = list(xs)
    return apply("concat", *parts, axis=_normalize_axis(parts[0], axis))


def stack(xs, axis=0):
    lifted = [expand_dims(x, axis) for x in xs]
    return concatenate(lifted, axis)


def flip(x, axis=-1):
    at = _normalize_axis(x, axis)
    return take(x, tensor(list(range(x.shape[at]))[::-1], "int32"), at)


# ---- selection ----

def take(x, idx, axis=0):
    """Rows of `x` along `axis` picked by int32 indices; the index shape replaces that axis.
    Indices out of range are clamped (validation reports them)."""
    return apply("take", x, _as_index(idx), axis=_normalize_axis(x, axis))


def _along_last(x, axis, fn):
    """`fn` applied with `axis` moved to the end, and the result moved back."""
    at = _normalize_axis(x, axis)
    if at == x.ndim - 1:
        return fn(x)
    return swapaxes(fn(swapaxes(x, at, -1)), at, -1)


def take_along_axis(x, idx, axis=-1):
    """One element of `x` per entry of `idx`, which matches `x` except along `axis`."""
    idx = _as_index(idx)
    at = _normalize_axis(x, axis)
    if at == x.ndim - 1:
        return apply("take_along", x, idx)
    return swapaxes(apply("take_along", swapaxes(x, at, -1), swapaxes(idx, at, -1)), at, -1)


def argmax(x, axis=-1):
    """Position of the largest value along `axis` (int32); `axis=None` looks at every element."""
    if axis is None:
        return apply("argmax", x.reshape(-1))
    at = _normalize_axis(x, axis)
    return apply("argmax", x if at == x.ndim - 1 else swapaxes(x, at, -1))


def top_k(x, k, axis=-1):
    """The `k` largest values along `axis`, descending, and their int32 positions. Ties keep
    position order; NaN sorts last."""
    positions = _along_last(x, axis, lambda v: apply("arg_top_k", v, k=k))
    return take_along_axis(x, positions, axis), positions


def argsort(x, axis=-1, descending=False):
    """Positions that sort `x` along `axis`; stable, NaN last either way."""
    n = x.shape[_normalize_axis(x, axis)]
    return _along_last(x if descending else -x, axis, lambda v: apply("arg_top_k", v, k=n))


def sort(x, axis=-1, descending=False):
    """`x` sorted along `axis`; each value's gradient goes back to where it came from."""
    order = argsort(x, axis, descending)
    return take_along_axis(x, order, axis)


def cumsum(x, axis=-1):
    return _along_last(x, axis, lambda v: apply("cumsum", v, reverse=False))


# ---- reductions as functions ----

def sum(x, axis=None, keepdims=False):
    return x.sum(axis, keepdims)


def mean(x, axis=None, keepdims=False):
    return x.mean(axis, keepdims)


def max(x, axis=None, keepdims=False):
    return x.max(axis, keepdims)


def min(x, axis=None, keepdims=False):
    return x.min(axis, keepdims)


def var(x, axis=None, keepdims=False):
    return x.var(axis, keepdims)


def std(x, axis=None, keepdims=False):
    return x.std(axis, keepdims)


# ---- constant tensors ----

def zeros(shape, dtype="float32"):
    return filled(shape, 0, dtype)


def ones(shape, dtype="float32"):
    return filled(shape, 1, dtype)


def full(shape, value, dtype="float32"):
    return filled(shape, value, dtype)


def zeros_like(x):
    return filled(x.shape, 0, x.dtype)


def ones_like(x):
    return filled(x.shape, 1, x.dtype)


def arange(n, dtype="int32"):
    return _from_array(np.arange(n), dtype)


def linspace(start, stop, num, dtype="float32"):
    """`num` evenly spaced values from `start` to `stop` inclusive (start + i * step in float64,
    then rounded to `dtype`)."""
    spacing = 0.0 if num <= 1 else (stop - start) / (num - 1)
    return _from_array(np.array([start + i * spacing for i in range(num)], dtype=np.float64), dtype)


def eye(n, dtype="float32"):
    return _from_array(np.eye(n), dtype)


def tril(n, dtype="float32"):
    """The n x n lower triangle of ones (diagonal included): a causal attention mask."""
    return _from_array(np.tril(np.ones((n, n))), dtype)
