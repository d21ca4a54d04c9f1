"""Python indexing of tensors and tracers: `x[i]`, `x[a:b, ..., None]`, `x[::2]`, `x[idx]`.

Basic indices become one `slice` node (plus a reshape that drops integer-indexed axes and adds
`None` axes); a slice with a step other than 1 becomes a `take` of the positions it visits; an
index tensor, array or list selects along the first axis with `take`. The accepted forms and the
INVALID_SLICE diagnostics follow the reference's `_Ops.__getitem__` (python/rg/_core.py).
"""

import numpy as np

from .tensor import Tensor, Tracer, error, tensor


def _is_index_array(key):
    return isinstance(key, (Tensor, Tracer, list, np.ndarray))


def _expand_ellipsis(x, items):
    dots = [i for i, k in enumerate(items) if k is Ellipsis]
    if not dots:
        return items
    named = sum(1 for k in items if k is not None and k is not Ellipsis)
    at = dots[0]
    return items[:at] + [slice(None)] * max(0, x.ndim - named) + items[at + 1:]


def index(x, key):
    from .ops import take
    if _is_index_array(key):
        return take(x, tensor(key, "int32") if isinstance(key, list) else key, 0)
    items = _expand_ellipsis(x, list(key) if isinstance(key, tuple) else [key])
    if sum(1 for k in items if k is not None) > x.ndim:
        raise error("INVALID_SLICE", {"shape": x.shape, "index_rank": len(items)}, "too_many_indices")
    # Pad with full slices for the trailing axes.
    items += [slice(None)] * (x.ndim - sum(1 for k in items if k is not None))

    # Strided slices first: each becomes a take along its axis, then a plain full slice.
    axis = 0
    for pos, k in enumerate(items):
        if k is None:
            continue
        if isinstance(k, slice) and k.step not in (None, 1):
            picks = range(*k.indices(x.shape[axis]))
            if len(picks) == 0:
                raise error("INVALID_SLICE", {"shape": x.shape, "axis": axis, "slice": repr(k)}, "stepped_slice_selects_nothing")
            x = take(x, tensor(list(picks), "int32"), axis)
            items[pos] = slice(None)
        axis += 1

    starts, stops, out_shape = [], [], []
    axis = 0
    for k in items:
        if k is None:
            out_shape.append(1)
            continue
        dim = x.shape[axis]
        if isinstance(k, slice):
            lo, hi, _ = k.indices(dim)
            hi = max(lo, hi)
            starts.append(lo)
            stops.append(hi)
            out_shape.append(hi - lo)
        elif isinstance(k, (int, np.integer)):
            at = int(k) + dim if k < 0 else int(k)
            if not 0 <= at < dim:
                raise error("INVALID_SLICE", {"shape": x.shape, "axis": axis, "index": int(k)}, "index_out_of_bounds")
            starts.append(at)
            stops.append(at + 1)
        else:
            raise error("INVALID_SLICE", {"shape": x.shape, "index_type": type(k).__name__}, "unsupported_index_type")
        axis += 1
    from .tensor import apply
    out = apply("slice", x, starts=starts, stops=stops)
    return out if tuple(out_shape) == out.shape else out.reshape(out_shape)
