"""Checkpoints of trees of tensors in the safetensors format: nothing is unpickled or executed
when a file is read.

The layout is the reference's (python/rg/checkpoint.py:37-105), so checkpoints move between the
two: an 8-byte little-endian header length, a JSON header naming every tensor by its dotted tree
path (dtype code, shape, byte range in the data section), then the raw little-endian data. The
header's `__metadata__` holds the user's string metadata and, under `rg_tree`, the tree's
structure as nested JSON lists, so `load` rebuilds the same tuples, lists and dicts. A file
written by another tool (no `rg_tree`) loads as a flat dict of its names.

Writes are atomic: the file is written beside its target, flushed to disk, and renamed over it,
so a crash leaves the previous checkpoint intact.
"""

import json
import os
import struct

import numpy as np

from . import _pytree
from ._native import _rg
from .tensor import Tensor, tensor

_CODE = {"float32": "F32", "float64": "F64", "int32": "I32"}
_DTYPE = {code: name for name, code in _CODE.items()}
_WIDTH = {"F32": 4, "F64": 8, "I32": 4}
_HEADER_LIMIT = 100 << 20
_TREE_KEY = "rg_tree"


def _treedef_to_json(d):
    """A TreeDef as the nested lists the format stores: null for a leaf, ["none"], a container
    kind with its children, and for a dict the kind, its keys and its children."""
    if d.kind == "leaf":
        return None
    if d.kind == "none":
        return ["none"]
    children = [_treedef_to_json(c) for c in d.children]
    return ["dict", list(d.keys), children] if d.kind == "dict" else [d.kind, children]


def _treedef_from_json(j):
    if j is None:
        return _pytree.LEAF
    if not isinstance(j, list) or not j:
        raise ValueError("malformed tree structure")
    if j[0] == "none":
        return _pytree.TreeDef("none")
    if j[0] == "dict":
        return _pytree.TreeDef("dict", j[1], [_treedef_from_json(c) for c in j[2]])
    if j[0] in ("tuple", "list"):
        return _pytree.TreeDef(j[0], (), [_treedef_from_json(c) for c in j[1]])
    raise ValueError(f"unknown container kind {j[0]!r}")


def _names(treedef):
    """Stored names of a tree's leaves in leaf order; a bare leaf is stored as `value`."""
    return [name or "value" for name in treedef.paths()]


def save(path, tree, metadata=None):
    """Writes `tree` (tensors, arrays or numbers in tuples, lists and dicts) to `path`.
    `metadata` is an optional dict of strings kept in the file."""
    leaves, treedef = _pytree.flatten(tree)
    tensors = [tensor(leaf) for leaf in leaves]
    extra = dict(metadata or {})
    for key, value in extra.items():
        if not isinstance(value, str):
            raise TypeError(f"checkpoint metadata {key!r} must be a string")
    header = {}
    offset = 0
    for name, t in zip(_names(treedef), tensors):
        size = t.size * _WIDTH[_CODE[t.dtype]]
        header[name] = {"dtype": _CODE[t.dtype], "shape": list(t.shape), "data_offsets": [offset, offset + size]}
        offset += size
    extra[_TREE_KEY] = json.dumps(_treedef_to_json(treedef))
    header["__metadata__"] = extra
    head = json.dumps(header).encode()
    staging = f"{path}.tmp.{os.getpid()}"
    try:
        with open(staging, "wb") as f:
            f.write(struct.pack("<Q", len(head)))
            f.write(head)
            for t in tensors:
                f.write(t._t.tobytes())
            f.flush()
            os.fsync(f.fileno())
        os.replace(staging, path)
    finally:
        if os.path.exists(staging):
            os.remove(staging)


def load(path, with_metadata=False):
    """Reads a checkpoint: the saved tree (or, for a file without tree structure, a flat dict
    of names), and with `with_metadata` also the user metadata. Raises ValueError on a
    truncated, oversized or inconsistent file."""
    with open(path, "rb") as f:
        raw = f.read()
    if len(raw) < 8:
        raise ValueError(f"{path}: not a safetensors file (truncated header)")
    (head_len,) = struct.unpack("<Q", raw[:8])
    if head_len > _HEADER_LIMIT or 8 + head_len > len(raw):
        raise ValueError(f"{path}: header of {head_len} bytes does not fit the file")
    try:
        header = json.loads(raw[8:8 + head_len])
    except ValueError as e:
        raise ValueError(f"{path}: header is not JSON ({e})") from None
    meta = header.pop("__metadata__", {}) or {}
    data = memoryview(raw)[8 + head_len:]
    stored = {}
    for name, info in header.items():
        code = info.get("dtype")
        if code not in _DTYPE:
            raise ValueError(f"{path}: tensor {name!r} has unsupported dtype {code}")
        shape = [int(d) for d in info["shape"]]
        start, end = info["data_offsets"]
        want = _WIDTH[code] * int(np.prod(shape, dtype=np.int64))
        if not 0 <= start <= end <= len(data) or end - start != want:
            raise ValueError(f"{path}: tensor {name!r} has offsets that do not match its shape or the file")
        stored[name] = Tensor(_rg.Tensor(bytes(data[start:end]), shape, _DTYPE[code]))
    user = {k: v for k, v in meta.items() if k != _TREE_KEY}
    if _TREE_KEY in meta:
        treedef = _treedef_from_json(json.loads(meta[_TREE_KEY]))
        names = _names(treedef)
        if sorted(names) != sorted(stored):
            raise ValueError(f"{path}: the stored tree structure does not match the stored tensors")
        result = _pytree.unflatten(treedef, [stored[n] for n in names])
    else:
        result = stored
    return (result, user) if with_metadata else result
