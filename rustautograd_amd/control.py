"""Control flow inside traced functions: `scan`, `while_loop` and `cond`.

Each traces its body functions into sub-graphs of one node of the enclosing graph (the
reference's python/rg/_core.py:388-503 and src/plan.rs:737-831).
"""

from .tensor import error


def _unsupported(what):
    raise error("UNSUPPORTED_OPERATION", {"operation": what}, "control_flow_is_not_part_of_the_hip_backend_yet")


def scan(f, init, xs=None, length=None):
    """`carry, y = f(carry, x)` over the first axis of `xs`; returns (carry, stacked ys)."""
    _unsupported("scan")


def while_loop(cond_fn, body_fn, init, max_iterations=100000):
    """`state = body_fn(state)` while `cond_fn(state)` is nonzero."""
    _unsupported("while_loop")


def cond(pred, true_fn, false_fn, *args):
    """`true_fn(*args)` if `pred` is nonzero, else `false_fn(*args)`; only one branch runs."""
    _unsupported("cond")
