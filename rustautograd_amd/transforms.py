"""Function transformations: reverse-mode gradients, forward-mode products, Hessians and
hand-written gradient rules. They work on traced functions: inside `compile` they add nodes to
the graph being traced (the engine's autodiff, csrc/engine/autodiff.cpp, differentiates); called
on concrete tensors they compile themselves once and run. Signatures and results follow the
reference's python/rg/_core.py (`value_and_grad`, `grad`, `jvp`, `hessian`, `custom_vjp`).
"""

from . import _pytree
from .tensor import TRACES, Tensor, Tracer, caller_source, error, first_dtype, lift
from .ops import stack, zeros_like


def _run_eagerly(fn, *args):
    from .program import compile
    return compile(fn, args, validate="none")(*args)


def _traced_or_eager(fn):
    """`fn` itself inside a trace; outside one, `fn` compiled for these arguments and run."""
    def wrapper(*args):
        return fn(*args) if TRACES.active else _run_eagerly(fn, *args)
    return wrapper


def _as_tracers(graph, tree):
    """The leaves of `tree` as tracers of `graph` (tensors and numbers become constants), and the
    tree's structure."""
    leaves, treedef = _pytree.flatten(tree)
    dtype = first_dtype(leaves) or "float32"
    return [Tracer(graph, lift(graph, leaf, dtype)) for leaf in leaves], treedef


def value_and_grad(f, argnums=0, has_aux=False):
    """`f(*args) -> scalar` becomes `(*args) -> (value, gradients)`, the gradients having the
    structure of `args[argnums]` (a tuple of them when `argnums` is a tuple). With `has_aux`, `f`
    returns `(scalar, aux)` and the value is `(scalar, aux)`."""
    several = isinstance(argnums, tuple)
    positions = argnums if several else (argnums,)

    def differentiated(*args):
        if not TRACES.active:
            return _run_eagerly(differentiated, *args)
        g = TRACES.graph
        where = caller_source()
        call_args = list(args)
        wrt = []
        for pos in positions:
            tracers, treedef = _as_tracers(g, args[pos])
            call_args[pos] = _pytree.unflatten(treedef, tracers)
            wrt.append((tracers, treedef))
        result = f(*call_args)
        value, aux = result if has_aux else (result, None)
        if not isinstance(value, (Tensor, Tracer, int, float)):
            raise error("GRAD_NON_SCALAR", {"returned_type": type(value).__name__}, "function_must_return_a_scalar_tensor")
        all_wrt = [t for tracers, _ in wrt for t in tracers]
        y = lift(g, value, first_dtype(all_wrt) or "float32")
        grads = []
        for tracers, treedef in wrt:
            ids = g.grad(y, [t._id for t in tracers], where)
            grads.append(_pytree.unflatten(treedef, [Tracer(g, i) for i in ids]))
        out_value = (Tracer(g, y), aux) if has_aux else Tracer(g, y)
        return out_value, (tuple(grads) if several else grads[0])

    return differentiated


def grad(f, argnums=0, has_aux=False):
    """The gradients of `value_and_grad`; with `has_aux`, `(gradients, aux)`."""
    with_value = value_and_grad(f, argnums, has_aux)

    def differentiated(*args):
        value, grads = with_value(*args)
        if has_aux:
            return grads, value[1]
        return grads

    return differentiated


def jvp(f, primals, tangents):
    """`(f(*primals), J tangents)`: the Jacobian-vector product, from the gradient of the
    vector-Jacobian product with respect to its cotangent (two reverse passes)."""

    def both(primals, tangents):
        g = TRACES.graph
        ys = f(*primals)
        cot = Tracer(g, lift(g, zeros_like(ys), ys.dtype))
        vjp = grad(lambda ps: (f(*ps) * cot).sum())(tuple(primals))
        pairs = zip(_pytree.leaves(vjp), _pytree.leaves(tuple(tangents)))
        total = None
        for a, b in pairs:
            term = (a * b).sum()
            total = term if total is None else total + term
        (jv,) = g.grad(total._id, [cot._id], caller_source())
        return ys, Tracer(g, jv)

    return _traced_or_eager(both)(tuple(primals), tuple(tangents))


def hessian(f):
    """The dense Hessian of a scalar function of one tensor, shape `x.shape + x.shape`."""

    def h(x):
        n = grad(f)(x).reshape(-1).shape[0]
        rows = [grad(lambda v, i=i: grad(f)(v).reshape(-1)[i])(x).reshape(-1) for i in range(n)]
        dims = tuple(x.shape)
        return stack(rows).reshape(dims + dims)

    return _traced_or_eager(h)


def custom_vjp(f, bwd):
    """`f` with a hand-written gradient: `bwd(args, y, cotangent)` returns one gradient per
    argument, each of its argument's shape and dtype."""

    def wrapped(*args):
        if not TRACES.active:
            return _run_eagerly(wrapped, *args)
        g = TRACES.graph
        where = caller_source()
        dtype = first_dtype(args) or "float32"
        inputs = [Tracer(g, lift(g, a, dtype)) for a in args]
        y = f(*inputs)
        cot = Tracer(g, g.placeholder(list(y.shape), y.dtype))
        grads = bwd(tuple(inputs), y, cot)
        if len(grads) != len(inputs):
            raise error("CUSTOM_VJP_MISMATCH", {"inputs": len(inputs), "gradients": len(grads)}, "rule_must_return_one_gradient_per_input")
        rules = []
        for x, gx in zip(inputs, grads):
            gx = gx if isinstance(gx, Tracer) else Tracer(g, lift(g, gx, x.dtype))
            if gx.shape != x.shape or gx.dtype != x.dtype:
                raise error("CUSTOM_VJP_MISMATCH", {"input_shape": x.shape, "gradient_shape": gx.shape, "input_dtype": x.dtype,
                                                    "gradient_dtype": gx.dtype}, "gradient_must_match_its_input")
            rules.append((x._id, gx._id))
        return Tracer(g, g.custom(y._id, cot._id, rules, where))

    return wrapped
