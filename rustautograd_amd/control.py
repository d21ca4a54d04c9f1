"""Control flow inside traced functions: `scan`, `while_loop` and `cond`.

Each traces its body functions into graphs of their own that become one node of the enclosing
graph (the reference's python/rg/_core.py:354-503; graph nodes src/graph.rs:101-109). A body
sees its declared arguments as its first inputs; any tracer of an enclosing trace it uses is
captured as a further input, so the node feeds the body (declared inputs, captures) in that order.
Called on concrete tensors, each compiles itself for these arguments and runs.
"""

from . import _pytree
from ._native import _rg
from .tensor import TRACES, Tracer, caller_source, error, first_dtype, lift, tracing


def _mismatch(part, want, got):
    return error("CONTROL_FLOW_SHAPE_MISMATCH", {"part": part, "expected": repr(want), "actual": repr(got)},
                 f"{part}_must_keep_its_structure_shape_and_dtype")


class _Body:
    """A body graph being traced inside `parent`, with the outer nodes it captured."""

    def __init__(self, parent, specs, where):
        self.parent = parent
        self.graph = _rg.Graph()
        self.where = where
        self.inputs = [self.graph.input(list(shape), dtype, where) for shape, dtype in specs]
        self.captures = []     # parent node ids, in the order of the body inputs they feed
        self._input_of = {}    # parent node id -> body input node

    def take(self, outer):
        """The body input fed by parent node `outer`, made on first use."""
        if outer not in self._input_of:
            self._input_of[outer] = self.graph.input(list(self.parent.shape(outer)), self.parent.dtype(outer), self.where)
            self.captures.append(outer)
        return self._input_of[outer]

    def capture(self, value):
        # Into the parent first: a tracer from further out is captured level by level.
        return self.take(lift(self.parent, value, value.dtype))

    def trace(self, fn, make_args):
        """Runs `fn(*make_args(input tracers))` into the body; returns (result ids, result structure)."""
        with tracing(self.graph, self.capture):
            out = fn(*make_args([Tracer(self.graph, i) for i in self.inputs]))
            leaves, out_def = _pytree.flatten(out)
            dtype = first_dtype(leaves) or "float32"
            ids = [lift(self.graph, leaf, dtype) for leaf in leaves]
        return ids, out_def

    def signature(self, ids):
        return [(tuple(self.graph.shape(i)), self.graph.dtype(i)) for i in ids]


def _lift_tree(graph, tree):
    leaves, treedef = _pytree.flatten(tree)
    dtype = first_dtype(leaves) or "float32"
    return [lift(graph, leaf, dtype) for leaf in leaves], treedef


def _specs(graph, ids, drop_leading=False):
    return [(tuple(graph.shape(i))[1:] if drop_leading else tuple(graph.shape(i)), graph.dtype(i)) for i in ids]


def _eagerly(fn, *args):
    from .program import compile
    return compile(fn, args, validate="none")(*args)


def scan(f, init, xs=None, length=None):
    """`carry, y = f(carry, x)` over the first axis of `xs`, in one graph node; returns
    `(final carry, stacked ys)`. Differentiable. Without `xs`, `length` gives the step count and
    `f` receives `None` as `x`; a body returning `None` as `y` makes the stacked ys `None`."""
    if not TRACES.active:
        if xs is None:
            return _eagerly(lambda c: scan(f, c, None, length), init)
        return _eagerly(lambda c, x: scan(f, c, x, length), init, xs)
    g = TRACES.graph
    where = caller_source()
    carry, c_def = _lift_tree(g, init)
    x_ids, x_def = _lift_tree(g, xs) if xs is not None else ([], None)
    lengths = {tuple(g.shape(i))[0] if g.shape(i) else None for i in x_ids}
    if length is not None:
        lengths.add(length)
    if len(lengths) != 1 or None in lengths:
        raise error("CONTROL_FLOW_SHAPE_MISMATCH", {"part": "xs", "lengths": repr(sorted(map(str, lengths)))},
                    "xs_need_one_shared_first_axis_or_an_explicit_length")
    n = lengths.pop()
    body = _Body(g, _specs(g, carry) + _specs(g, x_ids, drop_leading=True), where)

    def make_args(tracers):
        c = _pytree.unflatten(c_def, tracers[:len(carry)])
        x = _pytree.unflatten(x_def, tracers[len(carry):]) if xs is not None else None
        return c, x

    def step(c, x):
        out = f(c, x)
        if not (isinstance(out, tuple) and len(out) == 2):
            raise error("CONTROL_FLOW_SHAPE_MISMATCH", {"part": "body", "returned": type(out).__name__},
                        "scan_body_must_return_carry_and_y")
        new_c, y = out
        return new_c, (() if y is None else y)

    ids, out_def = body.trace(step, make_args)
    if out_def.children[0] != c_def:
        raise _mismatch("carry", c_def, out_def.children[0])
    n_c = len(carry)
    if body.signature(ids[:n_c]) != _specs(g, carry):
        raise _mismatch("carry", _specs(g, carry), body.signature(ids[:n_c]))
    node = g.scan(body.graph, ids, n_c, len(x_ids), n, carry + x_ids + body.captures, False, where)
    final = [Tracer(g, g.output(node, k, list(g.shape(i)), g.dtype(i), where)) for k, i in enumerate(carry)]
    stacked = [Tracer(g, g.output(node, n_c + k, [n] + list(shape), dtype, where))
               for k, (shape, dtype) in enumerate(body.signature(ids[n_c:]))]
    y_def = out_def.children[1]
    ys = None if y_def == _pytree.TreeDef("tuple") else _pytree.unflatten(y_def, stacked)
    return _pytree.unflatten(c_def, final), ys


def while_loop(cond_fn, body_fn, init, max_iterations=100000):
    """`state = body_fn(state)` while `cond_fn(state)` is nonzero, in one graph node. Not
    differentiable. Validation reports WHILE_LIMIT_REACHED when `max_iterations` stops the loop;
    `run` does not check and returns the state reached at the limit."""
    if not TRACES.active:
        return _eagerly(lambda s: while_loop(cond_fn, body_fn, s, max_iterations), init)
    g = TRACES.graph
    where = caller_source()
    state, s_def = _lift_tree(g, init)
    specs = _specs(g, state)

    def make_args(tracers):
        return (_pytree.unflatten(s_def, tracers[:len(state)]),)

    cond = _Body(g, specs, where)
    c_ids, _ = cond.trace(cond_fn, make_args)
    if len(c_ids) != 1 or tuple(cond.graph.shape(c_ids[0])) not in ((), (1,)):
        raise error("CONTROL_FLOW_SHAPE_MISMATCH", {"part": "condition", "outputs": [list(cond.graph.shape(i)) for i in c_ids]},
                    "condition_must_be_a_scalar")
    body = _Body(g, specs, where)
    for outer in cond.captures:  # the same captures first, in the same order
        body.take(outer)
    b_ids, b_def = body.trace(body_fn, make_args)
    if b_def != s_def:
        raise _mismatch("state", s_def, b_def)
    if body.signature(b_ids) != list(specs):
        raise _mismatch("state", list(specs), body.signature(b_ids))
    for outer in body.captures[len(cond.captures):]:  # captures of the body alone: unused by the condition
        cond.take(outer)
    node = g.while_loop(cond.graph, c_ids[0], body.graph, b_ids, len(state), max_iterations, state + body.captures, where)
    final = [Tracer(g, g.output(node, k, list(g.shape(i)), g.dtype(i), where)) for k, i in enumerate(state)]
    return _pytree.unflatten(s_def, final)


def cond(pred, true_fn, false_fn, *args):
    """`true_fn(*args)` if `pred` is nonzero, else `false_fn(*args)`; only the chosen branch runs
    (unlike `where`, which computes both). Differentiable. Both branches must return the same
    structure, shapes and dtypes."""
    if not TRACES.active:
        return _eagerly(lambda p, *a: cond(p, true_fn, false_fn, *a), pred, *args)
    g = TRACES.graph
    where = caller_source()
    arg_ids, a_def = _lift_tree(g, args)
    p_id = lift(g, pred, first_dtype([pred]) or "float32")
    specs = _specs(g, arg_ids)

    def make_args(tracers):
        return _pytree.unflatten(a_def, tracers[:len(arg_ids)])

    then_b = _Body(g, specs, where)
    t_ids, t_def = then_b.trace(true_fn, make_args)
    else_b = _Body(g, specs, where)
    for outer in then_b.captures:
        else_b.take(outer)
    e_ids, e_def = else_b.trace(false_fn, make_args)
    if t_def != e_def:
        raise _mismatch("branches", t_def, e_def)
    if then_b.signature(t_ids) != else_b.signature(e_ids):
        raise _mismatch("branches", then_b.signature(t_ids), else_b.signature(e_ids))
    for outer in else_b.captures[len(then_b.captures):]:
        then_b.take(outer)
    node = g.cond(then_b.graph, t_ids, else_b.graph, e_ids, [p_id] + arg_ids + else_b.captures, where)
    outs = [Tracer(g, g.output(node, k, list(shape), dtype, where)) for k, (shape, dtype) in enumerate(then_b.signature(t_ids))]
    return _pytree.unflatten(t_def, outs)
