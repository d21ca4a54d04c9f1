"""Compiling traced functions and running compiled training steps.

`compile` traces a Python function into the engine's graph, and the engine differentiates,
optimizes, plans and validates it for a device (csrc/engine/validate.cpp). `run` iterates a
compiled step `state -> new state` on the device, the whole loop in native code with no Python
between steps; `inspect` explains a compiled program or a finished run. The user-facing contract
(arguments, statuses, history names, diagnostics) is that of the reference's python/rg/_core.py
`compile`, `run` and `inspect` (lines 901-1135).
"""

import json
from typing import NamedTuple

from . import _native, _pytree
from ._native import _rg
from .ops import where
from .tensor import Tensor, Tracer, caller_source, diagnostic, error, first_dtype, lift, raise_record, tensor, tracing

DEFAULT_DEVICE = "hip"
MEMORY_WARNING_FRACTION = 0.5  # of the device's memory, for the planned intermediates


class Report(dict):
    """A JSON-compatible dict that prints as indented JSON. `repro_inputs` carries the tensors a
    replay found (they are not JSON)."""

    repro_inputs = None

    def __str__(self):
        return json.dumps(self, indent=2, ensure_ascii=False)

    @property
    def ok(self):
        return self.get("status") != "validation_failed"


class Signature:
    """The structure and per-leaf (shape, dtype) of a compiled program's inputs."""

    def __init__(self, treedef, specs):
        self.treedef = treedef
        self.specs = specs

    @classmethod
    def of(cls, args):
        leaves, treedef = _pytree.flatten(args)
        tensors = [tensor(leaf) for leaf in leaves]
        return cls(treedef, [(t.shape, t.dtype) for t in tensors]), tensors

    def child(self, k):
        return self.treedef.children[k]

    def mismatch(self, index, got):
        want = self.specs[index]
        return error("INPUT_SIGNATURE_MISMATCH", {"input_index": index, "expected": repr(want), "actual": repr(got),
                                                  "recompile_required": True}, "input_signature_changed")

    def natives(self, args):
        """The engine tensors of `args`, which must match this signature exactly."""
        got, tensors = Signature.of(args)
        if got.treedef != self.treedef:
            raise error("INPUT_SIGNATURE_MISMATCH", {"expected_structure": repr(self.treedef), "actual_structure": repr(got.treedef),
                                                     "recompile_required": True}, "input_structure_changed")
        if got.specs != self.specs:
            if len(got.specs) != len(self.specs):
                raise error("INPUT_SIGNATURE_MISMATCH", {"input_index": None, "expected": repr(self.specs), "actual": repr(got.specs),
                                                         "recompile_required": True}, "input_signature_changed")
            k = next(i for i, (a, b) in enumerate(zip(got.specs, self.specs)) if a != b)
            raise self.mismatch(k, got.specs[k])
        return [t._t for t in tensors]


class Compiled:
    """A program built for a device, with the report of its validation.

    Calling it runs one pass on concrete inputs of the example signature. The outputs of the
    function come first in the plan; `observe=True` instruments follow them."""

    def __init__(self, native, signature, out_def, n_user, instrument_names):
        self._n = native
        self._sig = signature
        self._out_def = out_def
        self._n_user = n_user
        self._extras = instrument_names
        self.report = Report(json.loads(native.report_json or "{}"))

    @property
    def device(self):
        return self._n.device

    def __call__(self, *inputs):
        outs = self._n.call(self._sig.natives(inputs))
        return _pytree.unflatten(self._out_def, [Tensor(t) for t in outs[:self._n_user]])

    def check(self, *args):
        """Runs the program instrumented on these inputs and reports what it found."""
        return Report(json.loads(self._n.check(self._sig.natives(args))))

    def profile(self, *inputs, repeats=5):
        """Device time of every plan step on these inputs, slowest first, plus a breakdown."""
        return Report(json.loads(self._n.profile(self._sig.natives(inputs), repeats)))

    def plan_summary(self):
        """One record per plan step: kind, operations, dtype, element count, shapes, slots."""
        return self._n.plan_summary()


def devices():
    """Device names `compile(device=...)` accepts in this process."""
    return list(_rg.available_devices())


# ---- observe=True: per-parameter statistics compiled into the program ---------------------------

def _instrument(graph, signature, inputs, out_leaves, out_def):
    """(name, node) pairs of scalars about each differentiated input: gradient norm, largest
    magnitude and fraction of exact zeros, the global gradient norm, and, when the step returns
    its state, each parameter's relative update size."""
    names = {t._id: p[2:] if p.startswith("0.") else p for t, p in zip(inputs, signature.treedef.paths())}
    last_grad = {}
    for _y, wrt, g in graph.grad_records():
        if wrt in names:
            last_grad[wrt] = g
    stats, squares = [], []
    for wrt, g in last_grad.items():
        gr = Tracer(graph, g)
        sq = (gr * gr).sum()
        squares.append(sq)
        stats.append((f"grad.{names[wrt]}.norm", sq.sqrt()))
        stats.append((f"grad.{names[wrt]}.max", abs(gr).max()))
        stats.append((f"grad.{names[wrt]}.zero", (0.0 >= abs(gr)).sum() / max(1, gr.size)))
    if squares:
        total = squares[0]
        for sq in squares[1:]:
            total = total + sq
        stats.append(("grad.global_norm", total.sqrt()))
    state_def = signature.child(0)
    if out_def == state_def or (_pytree.is_pair(out_def) and out_def.children[0] == state_def):
        n_state = state_def.n_leaves
        for before, after in zip(inputs[:n_state], out_leaves[:n_state]):
            if before._id in last_grad and isinstance(after, Tracer):
                delta = after - before
                size = (before * before).sum().sqrt()
                # A parameter at exactly zero records 0 (a ratio would be huge; NaN would stop the run).
                ratio = (delta * delta).sum().sqrt() / where(size > 0.0, size, 1.0)
                stats.append((f"update.{names[before._id]}", where(size > 0.0, ratio, 0.0)))
    return [(name, lift(graph, v, "float32")) for name, v in stats]


def compile(fn, example_inputs, validate="standard", device=None, optimize="search-linear", observe=False):
    """Traces `fn(*example_inputs)`; the engine differentiates, optimizes, plans and validates it
    for `device` (default "hip", the MI355X backend).

    `optimize`: "search-linear" (default; also reorders matrix products when cheaper, checked
    against the plain plan at validate="standard"), "standard", "search-exact", "search", "auto"
    or "none". `validate`: "none", "basic", "standard" or "thorough". `observe=True` adds
    per-parameter gradient and update statistics that `run` records in `history`.
    """
    device = device or DEFAULT_DEVICE
    args = example_inputs if isinstance(example_inputs, tuple) else (example_inputs,)
    signature, examples = Signature.of(args)
    graph = _rg.Graph()
    where_defined = caller_source()
    inputs = [Tracer(graph, graph.input(list(t.shape), t.dtype, where_defined)) for t in examples]
    with tracing(graph):
        out = fn(*_pytree.unflatten(signature.treedef, inputs))
        out_leaves, out_def = _pytree.flatten(out)
        dtype = first_dtype(examples) or "float32"
        out_ids = [lift(graph, leaf, dtype) for leaf in out_leaves]
        extras = _instrument(graph, signature, inputs, out_leaves, out_def) if observe else []
    if device not in devices():
        _native.require(device)
    native = _rg.compile(graph, out_ids + [node for _, node in extras], [t._t for t in examples], validate, device, optimize)
    compiled = Compiled(native, signature, out_def, len(out_ids), [name for name, _ in extras])
    _memory_warning(compiled, where_defined)
    return compiled


def _memory_warning(compiled, where_defined):
    """PLAN_NEAR_PHYSICAL_MEMORY when the plan's intermediates would fill much of the device."""
    capacity = _native.device_memory_bytes(compiled.device)
    planned = compiled.report.get("memory", {}).get("intermediate_bytes_planned", 0)
    if not capacity or planned <= capacity * MEMORY_WARNING_FRACTION:
        return
    record = diagnostic("PLAN_NEAR_PHYSICAL_MEMORY", {"intermediate_bytes_planned": planned, "physical_memory_bytes": capacity,
                                                      "warning_fraction": MEMORY_WARNING_FRACTION},
                        "plan_may_cause_swapping", certainty="suspected", severity="warning")
    record["node"]["source"] = where_defined
    compiled.report["diagnostics"].append(record)
    if compiled.report["status"] == "ok":
        compiled.report["status"] = "warning"


# ---- the step loop -----------------------------------------------------------------------------

class RunResult:
    """What `run` returns: `state`, the last `aux`, `history` (each scalar aux and instrument per
    step), `status` ("completed", "stopped_nonfinite", "stopped_by_callback"), `steps`,
    `requested_steps`, `nonfinite_step` and `elapsed` (seconds in the device step loop)."""

    def __init__(self, **fields):
        self.__dict__.update(fields)

    def __repr__(self):
        return f"rg.RunResult(status={self.status!r}, steps={self.steps}/{self.requested_steps}, elapsed={self.elapsed:.4f}s)"


class _Replay(NamedTuple):
    """Where the last chunk of a run started: enough for `inspect` to replay it."""
    spec: tuple          # (state_map, data_inputs, history outputs)
    state_def: object
    start: list          # engine tensors of the state at the chunk start
    batches: list        # the chunk's batches (engine tensors), in the order they were used
    ran: int             # steps the chunk ran
    offset: int          # steps completed before the chunk


class StepContract:
    """The rules a step function obeys to be `run`: it takes `state` or `(state, data)` and
    returns `new_state` or `(new_state, aux)`, the new state of the state's structure, shapes and
    dtypes (reference python/rg/_core.py `_setup`)."""

    def __init__(self, compiled, state):
        sig = compiled._sig
        arity = len(sig.treedef.children)
        if arity not in (1, 2):
            raise error("STATE_CONTRACT_VIOLATION", {"arity": arity}, "step_must_take_state_or_state_and_data")
        leaves, state_def = _pytree.flatten(state)
        if state_def != sig.child(0):
            raise error("INPUT_SIGNATURE_MISMATCH", {"expected_structure": repr(sig.child(0)), "actual_structure": repr(state_def),
                                                     "recompile_required": True}, "state_structure_changed")
        self.state = [tensor(leaf) for leaf in leaves]
        for k, t in enumerate(self.state):
            if (t.shape, t.dtype) != sig.specs[k]:
                raise sig.mismatch(k, (t.shape, t.dtype))
        out_def = compiled._out_def
        if out_def == state_def:
            self.aux_def = None
        elif _pytree.is_pair(out_def) and out_def.children[0] == state_def:
            self.aux_def = out_def.children[1]
        else:
            raise error("STATE_CONTRACT_VIOLATION", {"state_structure": repr(state_def), "output_structure": repr(out_def)},
                        "step_must_return_new_state_or_new_state_and_aux")
        self.compiled = compiled
        self.state_def = state_def
        self.n_state = len(self.state)
        self.data_def = sig.child(1) if arity == 2 else None

    def batch(self, data):
        """The engine tensors of one batch, checked against the data signature."""
        tensors = [tensor(leaf) for leaf in _pytree.leaves(data)]
        sig = self.compiled._sig
        for j, t in enumerate(tensors):
            if (t.shape, t.dtype) != sig.specs[self.n_state + j]:
                raise sig.mismatch(self.n_state + j, (t.shape, t.dtype))
        return [t._t for t in tensors]

    def batches(self, data):
        """(iterator or None, fixed list of batches) for the `data` argument of `run`."""
        if self.data_def is None:
            return None, []
        if callable(getattr(data, "__next__", None)):
            return data, []
        if _pytree.structure(data) == self.data_def:
            return None, [self.batch(data)]
        if isinstance(data, (list, tuple)) and data and all(_pytree.structure(b) == self.data_def for b in data):
            return None, [self.batch(b) for b in data]
        raise error("INPUT_SIGNATURE_MISMATCH", {"expected_batch_structure": repr(self.data_def),
                                                 "actual_structure": repr(_pytree.structure(data)), "recompile_required": True},
                    "data_structure_changed")

    def history_outputs(self):
        """{output index: history name}: the aux leaves holding one value, then the instruments."""
        named = {}
        if self.aux_def is not None:
            shapes = self.compiled._n.output_shapes
            for j, name in enumerate(self.aux_def.paths("aux")):
                k = self.n_state + j
                if all(d == 1 for d in shapes[k]):
                    named[k] = name
        for j, name in enumerate(self.compiled._extras):
            named[self.compiled._n_user + j] = name
        return named


def _first_error(report):
    for d in report["diagnostics"]:
        if d["severity"] == "error":
            return d
    return None


def run(compiled, state, data=None, steps=1, callback=None, every=None):
    """Runs `state = step(state[, data])` for `steps` steps on the device, with no Python between
    steps, and returns a RunResult.

    `data` is one batch, a list of batches (used in turn), or an iterator of batches (pulled
    `every` at a time, 256 by default). `callback(result)` is called every `every` steps with the
    result so far; returning False stops the run. The run stops after the first step whose new
    state or recorded history holds a non-finite value (status "stopped_nonfinite").
    """
    bad = _first_error(compiled.report)
    if bad is not None:
        raise_record(bad)
    contract = StepContract(compiled, state)
    iterator, fixed = contract.batches(data)
    named = contract.history_outputs()
    recorded = list(named)
    spec = ([(k, k) for k in range(contract.n_state)], list(range(contract.n_state, len(compiled._sig.specs))), recorded)
    if every:
        chunk = every
    else:
        chunk = steps if iterator is None else 256
    chunk = 1 if not steps else max(1, min(chunk, steps))

    history = {named[k]: [] for k in recorded}
    current = [t._t for t in contract.state]
    done, seconds, nonfinite, aux, stopped = 0, 0.0, None, None, False
    replay = _Replay(spec, contract.state_def, current, fixed[:1], 0, 0)
    while done < steps and nonfinite is None and not stopped:
        n = min(steps - done, chunk)
        if iterator is not None:
            part = []
            while len(part) < n:
                try:
                    part.append(contract.batch(next(iterator)))
                except StopIteration:
                    break
            if not part:
                break
            n = len(part)
        else:
            turn = done % len(fixed) if fixed else 0
            part = fixed[turn:] + fixed[:turn]
        new_state, outputs, hist, ran, bad_at, secs = compiled._n.run(*spec, current, part, n, True)
        replay = _Replay(spec, contract.state_def, current, part, ran, done)
        for k, values in zip(recorded, hist):
            history[named[k]].extend(values)
        done += ran
        seconds += secs
        if bad_at is not None:
            nonfinite = done - ran + bad_at
        elif not _rg.all_finite(new_state):
            nonfinite = done - 1
        current = new_state
        if contract.aux_def is not None and outputs:
            aux = _pytree.unflatten(contract.aux_def, [Tensor(t) for t in outputs[contract.n_state:compiled._n_user]])
        if callback is not None and nonfinite is None:
            so_far = _result(compiled, contract, current, aux, history, done, steps, None, seconds, replay, "running")
            stopped = callback(so_far) is False
    if nonfinite is not None:
        status = "stopped_nonfinite"
    elif stopped:
        status = "stopped_by_callback"
    else:
        status = "completed"
    if done == 0:
        aux, seconds = None, 0.0
    return _result(compiled, contract, current, aux, history, done, steps, nonfinite, seconds, replay, status)


def _result(compiled, contract, current, aux, history, done, steps, nonfinite, seconds, replay, status):
    return RunResult(status=status, state=_pytree.unflatten(contract.state_def, [Tensor(t) for t in current]), aux=aux,
                     history=history, steps=done, requested_steps=steps, nonfinite_step=nonfinite, elapsed=seconds,
                     compiled=compiled, _replay=replay)


def _finite_or_name(x):
    if x != x:
        return "nan"
    if x in (float("inf"), float("-inf")):
        return "inf" if x > 0 else "-inf"
    return x


def inspect(target):
    """A Compiled's validation report, or an account of a RunResult: a history summary, then
    either the instrumented check of the final state (gradient statistics and diagnostics) or,
    for a run stopped by a non-finite value, a replay of its last chunk to the first bad step
    and node, with the inputs that reproduce it (`repro_inputs`)."""
    if not isinstance(target, RunResult):
        return target.report
    r = target._replay
    c = target.compiled
    summary = {name: {"first": _finite_or_name(h[0]), "last": _finite_or_name(h[-1]), "min": _finite_or_name(min(h)),
                      "max": _finite_or_name(max(h))} for name, h in target.history.items() if h}
    out = Report(status=target.status, run={"steps": target.steps, "requested_steps": target.requested_steps,
                                            "elapsed_seconds": target.elapsed}, history=summary, diagnostics=[])
    if target.status != "stopped_nonfinite":
        if r.batches and r.ran:
            last_batch = r.batches[(r.ran - 1) % len(r.batches)]
        else:
            last_batch = r.batches[0] if r.batches else []
        final = json.loads(c._n.check([t._t for t in _pytree.leaves(target.state)] + last_batch))
        out.update(gradients=final["gradients"], diagnostics=final["diagnostics"])
        return out
    found = c._n.replay(*r.spec, r.start, r.batches, r.ran)
    if found is None:
        out.update(status="not_reproduced", diagnostics=[{"code": "REPLAY_DID_NOT_REPRODUCE", "severity": "warning",
                                                          "diagnosis": {"cause": "unknown", "certainty": "unknown"}}])
        return out
    bad_step, which_batch, state_before = found
    batch = r.batches[which_batch] if r.batches else []
    found_report = json.loads(c._n.check(state_before + batch))
    out.update(status="nonfinite_detected", diagnostics=found_report["diagnostics"])
    if all(d.get("severity") != "error" for d in out["diagnostics"]):
        # The unoptimized graph may stay finite where the optimized plan rounded over the edge.
        out["diagnostics"].append({"code": "NONFINITE_NOT_LOCALIZED", "severity": "warning",
                                   "diagnosis": {"cause": "reference_run_stayed_finite", "certainty": "unknown"}})
    out["repro"] = {"step": r.offset + bad_step, "batch_index": which_batch if r.batches else None,
                    "validate": c.report["repro"]["level"], "seed": c.report["repro"]["seed"]}
    data_def = c._sig.child(1) if len(c._sig.treedef.children) == 2 else None
    out.repro_inputs = {
        "state": _pytree.unflatten(r.state_def, [Tensor(t) for t in state_before]),
        "data": _pytree.unflatten(data_def, [Tensor(t) for t in batch]) if r.batches and data_def is not None else None,
    }
    return out
