"""Trees: nested tuples, lists and dicts of tensors, such as parameters and optimizer state.

Leaves are visited in a fixed order (dict keys sorted), which is the order of a compiled
program's inputs and of checkpoint entries. Names are dotted paths: `blocks.0.attn.qkv.w`.
"""

import builtins

from . import _pytree


def leaves(t):
    """The leaves of `t` in their fixed order."""
    return _pytree.leaves(t)


def structure(t):
    """A comparable description of `t` without its leaves."""
    return _pytree.structure(t)


def unflatten(structure_, values):
    """The tree of `structure_` holding `values` in leaf order."""
    return _pytree.unflatten(structure_, values)


def map(f, t, *rest):
    """`f` applied leaf by leaf to `t` and trees of the same structure."""
    vals, treedef = _pytree.flatten(t)
    columns = [vals]
    for other in rest:
        ov, od = _pytree.flatten(other)
        if od != treedef:
            raise ValueError("tree.map needs trees of the same structure")
        columns.append(ov)
    return _pytree.unflatten(treedef, [f(*row) for row in zip(*columns)])


def paths(t, prefix=""):
    """(name, leaf) pairs in leaf order; `prefix` is put before every name."""
    if t is None:
        return []
    vals, treedef = _pytree.flatten(t)
    names = treedef.paths()
    if treedef.kind == "leaf":
        return [(prefix[:-1] if prefix.endswith(".") else prefix, vals[0])]
    return [(prefix + name, v) for name, v in zip(names, vals)]


def size(t):
    """Number of elements over all leaves."""
    return builtins.sum(leaf.size for leaf in leaves(t))


def global_norm(t):
    """The L2 norm of all leaves taken together."""
    total = None
    for leaf in leaves(t):
        sq = (leaf * leaf).sum()
        total = sq if total is None else total + sq
    return total.sqrt()
