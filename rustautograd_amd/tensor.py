"""Values of the Python surface: concrete `Tensor`s, symbolic `Tracer`s, and the one primitive
(`apply`) through which every operation reaches the C++ engine.

Inside `compile` (or a transformation) operations record SSA nodes in the graph being traced;
outside they run eagerly: a one-operation graph is compiled for the default device and evaluated.
The operation names, attribute names and diagnostics are the engine's; the user-facing behaviour
follows the reference's python/rg/_core.py (`Tensor`, `Tracer`, `_Ops`, `tensor`).
"""

import json
import os
import sys

import numpy as np

from . import _native
from ._native import _rg, DiagnosticError

DTYPES = ("float32", "float64", "int32")
_HERE = os.path.dirname(os.path.abspath(__file__)) + os.sep


# ---- where user code called us, and structured errors -----------------------------------------

def caller_source():
    """`file:line` of the innermost stack frame outside this package: the user's own line."""
    frame = sys._getframe(1)
    while frame is not None and frame.f_code.co_filename.startswith(_HERE):
        frame = frame.f_back
    return None if frame is None else f"{frame.f_code.co_filename}:{frame.f_lineno}"


def diagnostic(code, observation, cause, certainty="verified", severity="error"):
    """A diagnostic record in the engine's schema (the reference's `Diag`, src/validate.rs)."""
    return {
        "status": "validation_failed" if severity == "error" else "warning", "severity": severity, "code": code,
        "node": {"id": None, "operation": None, "source": caller_source(), "role": "forward"},
        "observation": observation, "diagnosis": {"cause": cause, "certainty": certainty},
    }


def error(code, observation, cause, certainty="verified"):
    """A DiagnosticError carrying its record as `.diagnostic`."""
    record = diagnostic(code, observation, cause, certainty)
    exc = DiagnosticError(json.dumps(record))
    exc.diagnostic = record
    return exc


def raise_record(record):
    exc = DiagnosticError(json.dumps(record))
    exc.diagnostic = record
    raise exc


# ---- tracing state ------------------------------------------------------------------------------

class TraceStack:
    """Graphs being traced, innermost last. A graph on the stack receives every operation on
    tracers of its own; tracers of outer graphs reaching an inner one are captured by `lift`
    through the inner graph's `capture` hook (control-flow bodies), or refused."""

    def __init__(self):
        self.frames = []

    def push(self, graph, capture=None):
        self.frames.append((graph, capture))

    def pop(self):
        self.frames.pop()

    @property
    def active(self):
        return bool(self.frames)

    @property
    def graph(self):
        return self.frames[-1][0]

    def capture_hook(self, graph):
        for g, hook in reversed(self.frames):
            if g is graph:
                return hook
        return None

    def depth_of(self, graph):
        for i, (g, _) in enumerate(self.frames):
            if g is graph:
                return i
        return -1


TRACES = TraceStack()


class tracing:
    """Context manager: operations inside record nodes into `graph`."""

    def __init__(self, graph, capture=None):
        self.graph, self.capture = graph, capture

    def __enter__(self):
        TRACES.push(self.graph, self.capture)
        return self.graph

    def __exit__(self, *exc):
        TRACES.pop()
        return False


# ---- operators shared by tensors and tracers ----------------------------------------------------

# dunder -> (engine op, operand order): "ab" applies op(self, other), "ba" op(other, self).
_BINARY = {
    "add": ("add", "ab"), "radd": ("add", "ba"), "sub": ("sub", "ab"), "rsub": ("sub", "ba"),
    "mul": ("mul", "ab"), "rmul": ("mul", "ba"), "truediv": ("div", "ab"), "rtruediv": ("div", "ba"),
    "pow": ("pow", "ab"), "rpow": ("pow", "ba"), "matmul": ("matmul", "ab"), "rmatmul": ("matmul", "ba"),
    "gt": ("gt", "ab"), "ge": ("ge", "ab"), "lt": ("gt", "ba"), "le": ("ge", "ba"),
}
_UNARY_METHODS = ("exp", "log", "sqrt", "sin", "cos", "tanh", "floor")


def _binary_dunder(op, order):
    if order == "ab":
        return lambda self, other: apply(op, self, other)
    return lambda self, other: apply(op, other, self)


def _unary_method(op):
    def method(self):
        return apply(op, self)
    method.__name__ = op
    return method


class Value:
    """Methods common to `Tensor` and `Tracer`: arithmetic, reductions, shape manipulation and
    indexing. Subclasses provide `shape` and `dtype`."""

    __array_ufunc__ = None  # numpy hands mixed expressions to the reflected operators

    def __neg__(self):
        return apply("neg", self)

    def __abs__(self):
        return apply("abs", self)

    @property
    def ndim(self):
        return len(self.shape)

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    def _axis_list(self, axis):
        if axis is None:
            return list(range(self.ndim))
        picked = axis if isinstance(axis, (tuple, list)) else (axis,)
        return [a + self.ndim if a < 0 else a for a in picked]

    def _reduce(self, kind, axis, keepdims):
        return apply(kind, self, axes=self._axis_list(axis), keepdims=keepdims)

    def sum(self, axis=None, keepdims=False):
        return self._reduce("sum", axis, keepdims)

    def max(self, axis=None, keepdims=False):
        return self._reduce("max", axis, keepdims)

    def min(self, axis=None, keepdims=False):
        return self._reduce("min", axis, keepdims)

    def mean(self, axis=None, keepdims=False):
        axes = self._axis_list(axis)
        count = 1
        for a in axes:
            if 0 <= a < self.ndim:
                count *= self.shape[a]
        return self.sum(axis=axes, keepdims=keepdims) / count

    def var(self, axis=None, keepdims=False):
        centred = self - self.mean(axis=axis, keepdims=True)
        return (centred * centred).mean(axis=axis, keepdims=keepdims)

    def std(self, axis=None, keepdims=False):
        return self.var(axis=axis, keepdims=keepdims).sqrt()

    def reshape(self, *shape):
        dims = list(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else list(shape)
        if dims.count(-1) == 1:
            rest = int(np.prod([d for d in dims if d != -1], dtype=np.int64))
            dims[dims.index(-1)] = self.size // rest if rest else 0
        return apply("reshape", self, shape=dims)

    def transpose(self, *perm):
        order = list(perm[0]) if len(perm) == 1 and isinstance(perm[0], (tuple, list)) else list(perm)
        return apply("transpose", self, perm=order or list(range(self.ndim))[::-1])

    @property
    def T(self):
        return self.transpose()

    def cast(self, dtype):
        return apply("cast", self, dtype=dtype)

    def astype(self, dtype):
        return self if dtype == self.dtype else self.cast(dtype)

    def take(self, idx, axis=0):
        from .ops import take
        return take(self, idx, axis)

    def argmax(self, axis=-1):
        from .ops import argmax
        return argmax(self, axis)

    def swapaxes(self, a, b):
        from .ops import swapaxes
        return swapaxes(self, a, b)

    def squeeze(self, axis=None):
        from .ops import squeeze
        return squeeze(self, axis)

    def __iter__(self):
        if not self.shape:
            raise error("INVALID_SLICE", {"shape": self.shape}, "cannot_iterate_a_scalar")
        return (self[i] for i in range(self.shape[0]))

    def __getitem__(self, key):
        from .indexing import index
        return index(self, key)


for _name, (_op_name, _order) in _BINARY.items():
    setattr(Value, f"__{_name}__", _binary_dunder(_op_name, _order))
for _op_name in _UNARY_METHODS:
    setattr(Value, _op_name, _unary_method(_op_name))


class Tensor(Value):
    """A concrete value held by the engine (row-major bytes, a shape and a dtype)."""

    def __init__(self, native):
        self._t = native

    @property
    def shape(self):
        return tuple(self._t.shape)

    @property
    def dtype(self):
        return self._t.dtype

    def numpy(self):
        return np.frombuffer(self._t.tobytes(), dtype=self.dtype).reshape(self.shape).copy()

    def __array__(self, dtype=None, copy=None):
        out = self.numpy()
        return out if dtype is None else out.astype(dtype)

    def tolist(self):
        return self.numpy().tolist()

    def item(self):
        return int(self) if self.dtype == "int32" else float(self)

    def __float__(self):
        if self.size != 1:
            raise error("SHAPE_MISMATCH", {"shape": self.shape}, "scalar_conversion_of_non_scalar")
        return float(self.numpy().reshape(-1)[0])

    def __int__(self):
        return int(float(self))

    def __index__(self):
        if self.dtype != "int32" or self.size != 1:
            raise error("DTYPE_MISMATCH", {"dtype": self.dtype, "shape": self.shape}, "only_single_element_int32_converts_to_index")
        return int(self.numpy().reshape(-1)[0])

    def __bool__(self):
        return float(self) != 0.0

    def __repr__(self):
        return f"rg.Tensor({self.tolist()}, dtype={self.dtype})"


class Tracer(Value):
    """A symbolic value: node `_id` of graph `_g`, known by shape and dtype only."""

    def __init__(self, graph, node):
        self._g = graph
        self._id = node

    @property
    def shape(self):
        return tuple(self._g.shape(self._id))

    @property
    def dtype(self):
        return self._g.dtype(self._id)

    def _no_concrete(self, conversion):
        raise error("CONTROL_FLOW_ON_TRACER", {"node": self._id, "shape": self.shape, "conversion": conversion},
                    "python_value_depends_on_traced_tensor_use_rg_where")

    def __bool__(self):
        self._no_concrete("bool")

    def __float__(self):
        self._no_concrete("float")

    def __int__(self):
        self._no_concrete("int")

    def __index__(self):
        self._no_concrete("index")

    def __repr__(self):
        return f"rg.Tracer(node={self._id}, shape={self.shape}, dtype={self.dtype})"


# ---- making tensors -----------------------------------------------------------------------------

def _from_array(arr, dtype):
    arr = np.asarray(arr, dtype=dtype, order="C")
    return Tensor(_rg.Tensor(arr.tobytes(), list(arr.shape), dtype))


def tensor(data, dtype=None):
    """A Tensor from a Tensor, numpy array, number or nested list of numbers.

    Without `dtype`, integers (and booleans) give int32 and anything else float32; a numpy
    array already in float32, float64 or int32 keeps its dtype.
    """
    if isinstance(data, Tensor):
        return data if dtype in (None, data.dtype) else data.cast(dtype)
    if isinstance(data, Tracer):
        raise error("CONTROL_FLOW_ON_TRACER", {"node": data._id}, "tracer_used_as_concrete_data")
    if isinstance(data, np.ndarray) or (hasattr(data, "dtype") and hasattr(data, "tobytes")):
        arr = np.asarray(data)
        if dtype is None:
            dtype = str(arr.dtype) if str(arr.dtype) in DTYPES else ("int32" if arr.dtype.kind in "iub" else "float32")
        return _from_array(arr, dtype)
    try:
        arr = np.array(data, dtype=object if dtype is None else None)
    except ValueError:
        arr = None
    if arr is None or (arr.dtype == object and arr.shape and any(isinstance(x, (list, tuple)) for x in arr.reshape(-1))):
        raise error("SHAPE_MISMATCH", {"data": type(data).__name__}, "ragged_nested_sequence")
    if dtype is None:
        flat = arr.reshape(-1).tolist() if arr.dtype == object else None
        whole = flat is not None and all(isinstance(x, (int, np.integer)) for x in flat)
        dtype = "int32" if whole else "float32"
    if dtype == "int32":
        wide = np.asarray(arr.tolist() if arr.dtype == object else arr, dtype=np.int64)
        if wide.size and (wide.min() < -2 ** 31 or wide.max() >= 2 ** 31):
            raise error("DTYPE_MISMATCH", {"dtype": dtype}, "integer_out_of_int32_range")
        return _from_array(wide, dtype)
    return _from_array(np.asarray(arr.tolist() if arr.dtype == object else arr, dtype=np.float64), dtype)


def filled(shape, value, dtype="float32"):
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    return _from_array(np.full(shape, value, dtype=dtype), dtype)


# ---- the primitive ------------------------------------------------------------------------------

def first_dtype(values):
    """The dtype of the first Tensor or Tracer among `values` (numbers adopt it), or None."""
    for v in values:
        if isinstance(v, Value):
            return v.dtype
    return None


def lift(graph, value, dtype):
    """The node of `value` in `graph`: a tracer's own node, a captured outer tracer, or a
    constant holding a Tensor or a number (in `dtype`)."""
    if isinstance(value, Tracer):
        if value._g is graph:
            return value._id
        hook = TRACES.capture_hook(graph)
        if hook is not None and TRACES.depth_of(value._g) >= 0 and TRACES.depth_of(value._g) < TRACES.depth_of(graph):
            return hook(value)
        raise error("TRACER_LEAK", {"node": value._id}, "tracer_from_a_finished_trace")
    if isinstance(value, float) and dtype == "int32" and not value.is_integer():
        raise error("DTYPE_MISMATCH", {"scalar": value, "tensor_dtype": dtype}, "fractional_scalar_with_int32_tensor_cast_first")
    if not isinstance(value, Tensor):
        value = tensor(value, dtype if isinstance(value, (bool, int, float, np.number)) else None)
    return graph.constant(value._t, caller_source())


def apply(op, *args, **attrs):
    """One engine operation on tensors, tracers and numbers: a node of the innermost trace, or an
    eager evaluation on the default device."""
    dtype = first_dtype(args)
    where = caller_source()
    if TRACES.active:
        g = TRACES.graph
        ids = [lift(g, a, dtype) for a in args]
        return Tracer(g, g.op(op, ids, attrs or None, where))
    for a in args:
        if isinstance(a, Tracer):
            raise error("TRACER_LEAK", {"node": a._id}, "tracer_from_a_finished_trace")
    g = _rg.Graph()
    ids = [lift(g, a, dtype) for a in args]
    (out,) = g.eval([g.op(op, ids, attrs or None, where)])
    return Tensor(out)


def require_device(device):
    if device not in list(_rg.available_devices()):
        _native.require(device)
