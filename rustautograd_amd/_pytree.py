"""Nested containers of tensors ("trees"): flattening to leaves and a structure description.

Containers are tuples, lists and dicts; `None` is an empty container; anything else is a leaf.
Dict entries are visited in sorted key order, so a tree's leaf order (and with it the order of a
compiled program's inputs, outputs and checkpoint names) does not depend on insertion order, as
in the reference (python/rg/_core.py `_flatten`, python/rg/tree.py `paths`).
"""

_CONTAINERS = (tuple, list, dict)


class TreeDef:
    """The shape of a tree without its leaves. Two trees with equal TreeDefs hold leaves in the
    same positions; TreeDefs compare by value and hash, so they work as signature keys."""

    __slots__ = ("kind", "keys", "children")

    def __init__(self, kind, keys=(), children=()):
        self.kind = kind            # "leaf", "none", "tuple", "list" or "dict"
        self.keys = tuple(keys)     # dict keys, sorted
        self.children = tuple(children)

    def _ident(self):
        return (self.kind, self.keys, tuple(c._ident() for c in self.children))

    def __eq__(self, other):
        return isinstance(other, TreeDef) and self._ident() == other._ident()

    def __hash__(self):
        return hash(self._ident())

    def __repr__(self):
        if self.kind == "leaf":
            return "*"
        if self.kind == "none":
            return "None"
        if self.kind == "dict":
            return "{" + ", ".join(f"{k!r}: {c!r}" for k, c in zip(self.keys, self.children)) + "}"
        inner = ", ".join(repr(c) for c in self.children)
        return f"({inner},)" if self.kind == "tuple" and len(self.children) == 1 else ("(%s)" if self.kind == "tuple" else "[%s]") % inner

    @property
    def n_leaves(self):
        if self.kind == "leaf":
            return 1
        return sum(c.n_leaves for c in self.children)

    def labels(self):
        """Position labels of the direct children: dict keys, or indices as strings."""
        return list(self.keys) if self.kind == "dict" else [str(i) for i in range(len(self.children))]

    def paths(self, prefix=""):
        """Dotted names of the leaves in flatten order: `prefix`, `prefix.key`, `prefix.0.w`."""
        if self.kind == "leaf":
            return [prefix]
        out = []
        for label, child in zip(self.labels(), self.children):
            out.extend(child.paths(f"{prefix}.{label}" if prefix else label))
        return out


LEAF = TreeDef("leaf")


def flatten(tree):
    """(leaves, TreeDef) of a tree."""
    leaves = []

    def walk(node):
        if node is None:
            return TreeDef("none")
        if isinstance(node, dict):
            keys = sorted(node)
            return TreeDef("dict", keys, [walk(node[k]) for k in keys])
        if isinstance(node, (tuple, list)):
            return TreeDef("tuple" if isinstance(node, tuple) else "list", (), [walk(x) for x in node])
        leaves.append(node)
        return LEAF

    return leaves, walk(tree)


def unflatten(treedef, leaves):
    """Rebuilds the tree described by `treedef` from its leaves, in flatten order."""
    feed = iter(leaves)

    def build(d):
        if d.kind == "leaf":
            return next(feed)
        if d.kind == "none":
            return None
        parts = [build(c) for c in d.children]
        if d.kind == "dict":
            return dict(zip(d.keys, parts))
        return tuple(parts) if d.kind == "tuple" else parts

    return build(treedef)


def leaves(tree):
    return flatten(tree)[0]


def structure(tree):
    return flatten(tree)[1]


def is_pair(treedef):
    """True for a two-element tuple structure, the `(state, aux)` form of a step's result."""
    return treedef.kind == "tuple" and len(treedef.children) == 2
