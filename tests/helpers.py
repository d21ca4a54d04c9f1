"""Shared helpers: build a graph through the engine API, run it on a device, compare results."""

import numpy as np

import rustautograd_amd as rg
from rustautograd_amd import _rg


def t(a, dtype="float32"):
    return rg.tensor(np.asarray(a, dtype=dtype))


def seq(shape, dtype="float32"):
    """0.25 + |sin(0.73 i)|: positive, irregular values (the reference's tests/metal.rs:50-53)."""
    n = int(np.prod(shape)) if shape else 1
    return rg.tensor((0.25 + np.abs(np.sin(np.arange(n) * 0.73))).reshape(shape).astype(dtype))


def run_graph(device, build, inputs, optimize="none", n_out=None):
    """Traces `build(g, ids)` over fresh inputs, compiles it for `device` and calls it once."""
    g = _rg.Graph()
    ids = [g.input(list(x.shape), x.dtype) for x in inputs]
    out = build(g, ids)
    outs = out if isinstance(out, (list, tuple)) else [out]
    c = _rg.compile(g, list(outs), [x._t for x in inputs], "none", device, optimize)
    res = c.call([x._t for x in inputs])
    return [rg.Tensor(r).numpy() for r in res]


def op(g, name, ins, **attrs):
    return g.op(name, list(ins), attrs or None)


def ulp_distance(a, b):
    """Distance in units in the last place between float arrays of the same dtype (NaN == NaN)."""
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.float32:
        ia, ib = a.view(np.int32).astype(np.int64), b.view(np.int32).astype(np.int64)
        ia = np.where(ia < 0, np.int64(-(2 ** 31)) - ia, ia)
        ib = np.where(ib < 0, np.int64(-(2 ** 31)) - ib, ib)
    else:
        ia, ib = a.view(np.int64).astype(object), b.view(np.int64).astype(object)
        ia = np.array([(-(2 ** 63)) - x if x < 0 else x for x in ia.ravel()], dtype=object).reshape(a.shape)
        ib = np.array([(-(2 ** 63)) - x if x < 0 else x for x in ib.ravel()], dtype=object).reshape(b.shape)
    d = np.abs(ia - ib)
    both_nan = np.isnan(a) & np.isnan(b)
    return np.where(both_nan, 0, d)


def close(got, want, tol, what=""):
    """|got - want| <= tol * max(1, max|want|) elementwise, NaN matching NaN (tests/metal.rs:33-40)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    finite = want[np.isfinite(want)]
    scale = max(1.0, float(np.abs(finite).max())) if finite.size else 1.0
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    ok = same | (np.abs(got - want) <= tol * scale)
    if not ok.all():
        j = int(np.argmax(~ok.ravel()))
        raise AssertionError(f"{what}[{j}]: hip {got.ravel()[j]!r} cpu {want.ravel()[j]!r} (tol {tol} x {scale})")


def close_rel(got, want, tol, what=""):
    """|got - want| <= tol * max|want| elementwise: relative to the array's own largest magnitude
    (validate.rs:686-693 scales its device check the same way), so values well below 1 are not
    compared absolutely. An all-zero `want` needs `got` equal to it. Returns the largest
    difference in units of max|want|."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN positions differ"
    finite = np.isfinite(want)
    scale = float(np.abs(want[finite]).max()) if finite.any() else 0.0
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    diff = np.where(same, 0.0, np.abs(got - want))
    ok = diff <= tol * scale
    if not ok.all():
        j = int(np.argmax(~ok.ravel()))
        raise AssertionError(f"{what}[{j}]: hip {got.ravel()[j]!r} cpu {want.ravel()[j]!r} "
                             f"(tol {tol} x max|cpu| {scale:.3e}; worst {diff.max() / max(scale, 1e-300):.2e})")
    return float(diff.max() / scale) if scale > 0 else 0.0


def adamw_direction(mu, nu, count, b1, b2, eps):
    """AdamW's update direction from first and second moments after `count` steps, in float64
    (python/rg/optim.py:378-390 order): (mu / (1 - b1^t)) / (sqrt(nu / (1 - b2^t)) + eps)."""
    mu, nu = np.asarray(mu, np.float64), np.asarray(nu, np.float64)
    return (mu / (1.0 - b1 ** count)) / (np.sqrt(nu / (1.0 - b2 ** count)) + eps)


def updates_agree(old, hip, cpu, tol, what, adamw):
    """A parameter's update (new - old) on the device against the oracle's.

    `hip` and `cpu` are (new parameter, mu, nu, count) of one AdamW step from the same `old`
    parameter. AdamW divides each moment by the root of the second moment, so where a gradient
    element is near zero, rounding-level moment differences (checked separately, relative to
    each leaf's largest moment) become update differences up to the learning rate. The check
    therefore takes out what the two sides' own moments explain, computed in float64:
    |(dhip - dcpu) - lr (dir(cpu moments) - dir(hip moments))| <= tol * max|dcpu| + 2 ulp(new),
    the 2 ulp because new - old is formed from f32 values on both sides. A wrong update rule,
    bias correction or decay on either side fails it. Returns the worst residual beyond the 2 ulp
    allowance, in units of max|dcpu|."""
    p0 = np.asarray(old, np.float64)
    (p1, m1, v1, t1), (p2, m2, v2, t2) = hip, cpu
    assert float(t1) == float(t2), (what, t1, t2)
    d1, d2 = np.asarray(p1, np.float64) - p0, np.asarray(p2, np.float64) - p0
    lr = adamw["lr"]
    explained = lr * (adamw_direction(m2, v2, float(t2), adamw["b1"], adamw["b2"], adamw["eps"])
                      - adamw_direction(m1, v1, float(t1), adamw["b1"], adamw["b2"], adamw["eps"]))
    residual = np.abs((d1 - d2) - explained)
    scale = float(np.abs(d2).max())
    ulp = np.spacing(np.abs(np.asarray(p2, np.float32))).astype(np.float64)
    ok = residual <= tol * scale + 2.0 * ulp
    if not ok.all():
        j = int(np.argmax(~ok.ravel()))
        raise AssertionError(f"{what} update[{j}]: hip {d1.ravel()[j]!r} cpu {d2.ravel()[j]!r} explained "
                             f"{explained.ravel()[j]!r} (tol {tol} x max|dcpu| {scale:.3e})")
    return float(np.maximum(residual - 2.0 * ulp, 0.0).max() / scale) if scale > 0 else 0.0


def agree(build, inputs, tol=2e-6, what="", ulps=None):
    """Runs `build` on the HIP device and on the CPU oracle and compares every output."""
    hip = run_graph("hip", build, inputs)
    cpu = run_graph("cpu", build, inputs)
    for k, (a, b) in enumerate(zip(hip, cpu)):
        if ulps is not None and a.dtype in (np.float32, np.float64):
            d = ulp_distance(a, b)
            assert d.max() <= ulps, f"{what} output {k}: {int(d.max())} ulp apart; hip {a.ravel()[np.argmax(d)]} cpu {b.ravel()[np.argmax(d)]}"
        elif a.dtype == np.int32:
            assert np.array_equal(a, b), f"{what} output {k}: int32 results differ"
        else:
            close(a, b, tol, f"{what} output {k}")
    return hip, cpu


class G:
    """A graph under construction, in the vocabulary of the reference's tests/engine.rs:34-46."""

    def __init__(self):
        self.g = _rg.Graph()

    def input(self, shape, dtype="float64"):
        return self.g.input(list(shape), dtype)

    def const(self, values, shape=None, dtype="float64"):
        a = np.asarray(values, dtype=dtype)
        if shape is not None:
            a = a.reshape(shape)
        return self.g.constant(rg.tensor(a)._t)

    def scalar(self, v, dtype="float64"):
        return self.const(v, (), dtype)

    def op(self, name, ins, **attrs):
        return self.g.op(name, list(ins), attrs or None)

    def un(self, name, a, **attrs):
        return self.op(name, [a], **attrs)

    def bin(self, name, a, b):
        return self.op(name, [a, b])

    def sum_all(self, x):
        return self.op("sum", [x], axes=list(range(len(self.shape(x)))), keepdims=False)

    def grad(self, y, wrts):
        return list(self.g.grad(y, list(wrts)))

    def shape(self, x):
        return tuple(self.g.shape(x))

    def compile(self, outs, inputs, device="cpu", optimize="none", level="none"):
        return _rg.compile(self.g, list(outs), [rg.tensor(np.asarray(x))._t for x in inputs], level, device, optimize)

    def eval(self, outs, inputs=(), device="cpu", optimize="none"):
        """Compiles `outs` for `device` (the CPU oracle by default) and returns them as numpy arrays."""
        c = self.compile(outs, inputs, device, optimize)
        return [rg.Tensor(r).numpy() for r in c.call([rg.tensor(np.asarray(x))._t for x in inputs])]


def diag_code(excinfo):
    return excinfo.value.diagnostic["code"]


# ---- the device C ABI through ctypes (include/rg_hip.h) ----

import ctypes


class RunDesc(ctypes.Structure):
    """rg_run_desc of include/rg_hip.h."""
    _fields_ = [("n_swaps", ctypes.c_int64), ("swaps", ctypes.POINTER(ctypes.c_int64)),
                ("n_copies", ctypes.c_int64), ("copies", ctypes.POINTER(ctypes.c_int64)),
                ("n_data", ctypes.c_int64), ("data_slots", ctypes.POINTER(ctypes.c_int64)),
                ("data_bytes", ctypes.POINTER(ctypes.c_uint64)), ("n_batches", ctypes.c_int64),
                ("batches", ctypes.POINTER(ctypes.c_void_p)), ("n_history", ctypes.c_int64),
                ("history_slots", ctypes.POINTER(ctypes.c_int64)), ("steps", ctypes.c_int64),
                ("history", ctypes.POINTER(ctypes.c_double))]


class RunResult(ctypes.Structure):
    """rg_run_result of include/rg_hip.h."""
    _fields_ = [("done", ctypes.c_int64), ("nonfinite_step", ctypes.c_int64), ("seconds", ctypes.c_double)]


def plan_io(words):
    """Input slots and output slots of a flat plan (include/rg_plan.h: header, slots, consts,
    inputs, outputs)."""
    k = 2
    k += 1 + 3 * words[k]
    k += 1 + 3 * words[k]
    n = words[k]
    inputs = [words[k + 1 + 2 * j] for j in range(n)]
    k += 1 + 2 * n
    n = words[k]
    k += 1
    outputs = []
    for _ in range(n):
        outputs.append(words[k])
        k += 3 + words[k + 2]
    return inputs, outputs


def hip_abi():
    """librg_hip.so with argument and result types set for the entry points tests call."""
    from rustautograd_amd import _native
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    vp, i64, u64, cp, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t
    lib.rg_hip_program_new.restype = vp
    lib.rg_hip_program_new.argtypes = [ctypes.POINTER(i64), sz, cp, sz, cp, sz]
    lib.rg_hip_exec_new.restype = vp
    lib.rg_hip_exec_new.argtypes = [vp, cp, sz]
    for name in ("rg_hip_exec_free", "rg_hip_program_free", "rg_hip_program_inject_failure"):
        getattr(lib, name).argtypes = [vp]
    lib.rg_hip_program_inject_failure_after.argtypes = [vp, i64]
    lib.rg_hip_exec_write.argtypes = [vp, i64, vp, u64]
    lib.rg_hip_exec_read.argtypes = [vp, i64, vp, u64]
    for name in ("rg_hip_exec_run", "rg_hip_exec_run_noalloc"):
        getattr(lib, name).argtypes = [vp, ctypes.POINTER(RunDesc), ctypes.POINTER(RunResult)]
    lib.rg_hip_exec_failure.argtypes = [vp, cp, sz]
    return lib


def hip_program(lib, graph, outputs, optimize="none"):
    """A device program for `outputs` of `graph`, built through the C ABI: (handle, inputs, outputs)."""
    from rustautograd_amd import _rg
    words, blob = _rg.plan_words(graph, list(outputs), "hip", optimize)
    ins, outs = plan_io(words)
    arr = (ctypes.c_int64 * len(words))(*words)
    err = ctypes.create_string_buffer(4096)
    prog = lib.rg_hip_program_new(arr, len(words), blob, len(blob), err, len(err))
    assert prog, err.value
    return prog, ins, outs


def exec_failure(lib, e):
    msg = ctypes.create_string_buffer(1024)
    return msg.value.decode() if lib.rg_hip_exec_failure(e, msg, len(msg)) else None
