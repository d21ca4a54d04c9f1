"""rg_hip_exec_run_noalloc, the run loop that allocates nothing, against rg_hip_exec_run.

Two calls in a row through the C ABI, the second with smaller inputs: a gradient-descent program
with cycled batches, per-step history and buffer swaps, then a smaller one whose state is handed
back by copies. Each must give rg_hip_exec_run's state and history bit for bit. A run whose
buffers exceed the static scratch is refused before anything runs. A non-finite history value
stops both loops after the same step; an injected failure reports the steps a synchronization
confirmed, with and without history; run descriptions that do not fit the program are refused
by both entries before anything runs.
"""

import ctypes

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import _rg

from helpers import RunDesc, RunResult, exec_failure, hip_abi, hip_program, op

pytestmark = pytest.mark.gpu


def _gd_program(lib, rows, twin):
    """w <- w - 0.01 * grad(mean((x @ w - y)^2)); with `twin`, the state is (w, w2) and both take
    the new w (the output slot is shared, so the handoff copies)."""
    g = _rg.Graph()
    w = g.input([8], "float32")
    w2 = g.input([8], "float32") if twin else None
    x, y = g.input([rows, 8], "float32"), g.input([rows], "float32")
    err = op(g, "sub", [op(g, "matmul", [x, w]), y])
    loss = op(g, "div", [op(g, "sum", [op(g, "mul", [err, err])], axes=[0], keepdims=False),
                         g.constant(rg.tensor(np.float32(rows))._t)])
    grad = g.grad(loss, [w])[0]
    nw = op(g, "sub", [w, op(g, "mul", [grad, g.constant(rg.tensor(np.float32(0.01))._t)])])
    outs = [nw, nw, loss] if twin else [nw, loss]
    return hip_program(lib, g, outs)


def _run(lib, entry, prog, ins, outs, twin, batches, steps):
    """One run through `entry` from w = 0.1 * arange(8); returns (rc, result, state words, history)."""
    err = ctypes.create_string_buffer(4096)
    e = lib.rg_hip_exec_new(prog, err, len(err))
    assert e, err.value
    try:
        n_state = 2 if twin else 1
        w0 = (np.arange(8, dtype=np.float32) * 0.1).astype(np.float32)
        for k in range(n_state):
            assert lib.rg_hip_exec_write(e, ins[k], w0.ctypes.data, 32) == 0
        data_slots = (ctypes.c_int64 * 2)(ins[n_state], ins[n_state + 1])
        data_bytes = (ctypes.c_uint64 * 2)(batches[0][0].nbytes, batches[0][1].nbytes)
        ptrs = (ctypes.c_void_p * (2 * len(batches)))(*[a.ctypes.data for b in batches for a in b])
        hs = (ctypes.c_int64 * 1)(outs[-1])
        hist = (ctypes.c_double * steps)()
        if twin:
            cp = (ctypes.c_int64 * 6)(ins[0], outs[0], 8, ins[1], outs[1], 8)
            d = RunDesc(n_copies=2, copies=cp)
        else:
            sw = (ctypes.c_int64 * 2)(ins[0], outs[0])
            d = RunDesc(n_swaps=1, swaps=sw)
        d.n_data, d.data_slots, d.data_bytes = 2, data_slots, data_bytes
        d.n_batches, d.batches = len(batches), ptrs
        d.n_history, d.history_slots, d.steps, d.history = 1, hs, steps, hist
        res = RunResult()
        rc = getattr(lib, entry)(e, ctypes.byref(d), ctypes.byref(res))
        state = []
        for k in range(n_state):
            got = np.zeros(8, np.float32)
            assert lib.rg_hip_exec_read(e, ins[k], got.ctypes.data, 32) == 0
            state.append(got.view(np.uint32).copy())
        return rc, res, state, np.array(hist[:res.done]), exec_failure(lib, e)
    finally:
        lib.rg_hip_exec_free(e)


def _batches(rows, count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        x = rng.normal(size=(rows, 8)).astype(np.float32)
        out.append((x, (x @ np.arange(8, dtype=np.float32)).astype(np.float32)))
    return out


def test_noalloc_run_equals_the_run_loop_twice_with_a_smaller_second_input():
    lib = hip_abi()
    for rows, count, twin, steps in ((256, 3, False, 40), (64, 2, True, 25)):
        print(f"noalloc vs run: rows={rows} batches={count} copies={twin} steps={steps}", flush=True)
        prog, ins, outs = _gd_program(lib, rows, twin)
        try:
            batches = _batches(rows, count, rows)
            rc_ref, ref, state_ref, hist_ref, f_ref = _run(lib, "rg_hip_exec_run", prog, ins, outs, twin, batches, steps)
            rc, got, state, hist, f = _run(lib, "rg_hip_exec_run_noalloc", prog, ins, outs, twin, batches, steps)
            assert rc_ref == 0 and rc == 0, (f_ref, f)
            assert got.done == ref.done == steps and got.nonfinite_step == ref.nonfinite_step == -1
            for a, b in zip(state, state_ref):
                assert np.array_equal(a, b)
            assert np.array_equal(hist.view(np.uint64), hist_ref.view(np.uint64))
            assert hist[-1] < hist[0]
        finally:
            lib.rg_hip_program_free(prog)


def test_noalloc_run_refuses_buffers_beyond_the_static_scratch():
    lib = hip_abi()
    prog, ins, outs = _gd_program(lib, 256, False)
    try:
        one = _batches(256, 1, 0)[0]
        many = [one] * 4200  # 4200 cycled batches of 9 KiB: more than the 32 MiB of scratch
        rc, res, state, _, failure = _run(lib, "rg_hip_exec_run_noalloc", prog, ins, outs, False, many, 3)
        assert rc == -1 and res.done == 0
        assert "static scratch holds" in failure, failure
        w0 = (np.arange(8, dtype=np.float32) * 0.1).astype(np.float32)
        assert np.array_equal(state[0], w0.view(np.uint32))
    finally:
        lib.rg_hip_program_free(prog)


def _doubling_program(lib):
    """w <- 2 w, history sum(w): from w = 1e37 * (1, 2, 3, 4) the history overflows to inf."""
    g = _rg.Graph()
    w = g.input([4], "float32")
    nw = op(g, "mul", [w, g.constant(rg.tensor(np.float32(2.0))._t)])
    return hip_program(lib, g, [nw, op(g, "sum", [nw], axes=[0], keepdims=False)])


def _doubling_run(lib, entry, prog, win, wout, lout, steps, history, fail_after=None, x0=(1e37, 2e37, 3e37, 4e37)):
    err = ctypes.create_string_buffer(4096)
    e = lib.rg_hip_exec_new(prog, err, len(err))
    assert e, err.value
    try:
        x0 = np.array(x0, np.float32)
        assert lib.rg_hip_exec_write(e, win, x0.ctypes.data, 16) == 0
        swaps = (ctypes.c_int64 * 2)(win, wout)
        hs = (ctypes.c_int64 * 1)(lout)
        hist = (ctypes.c_double * steps)()
        d = RunDesc(n_swaps=1, swaps=swaps, n_history=1 if history else 0, history_slots=hs, steps=steps, history=hist)
        if fail_after is not None:
            lib.rg_hip_program_inject_failure_after(prog, fail_after)
        res = RunResult()
        rc = getattr(lib, entry)(e, ctypes.byref(d), ctypes.byref(res))
        got = np.zeros(4, np.float32)
        assert lib.rg_hip_exec_read(e, win, got.ctypes.data, 16) == 0
        return rc, res, got, np.array(hist[:res.done]), exec_failure(lib, e)
    finally:
        lib.rg_hip_exec_free(e)


def test_noalloc_stops_after_the_first_nonfinite_step_as_the_run_loop_does():
    lib = hip_abi()
    prog, (win,), (wout, lout) = _doubling_program(lib)
    try:
        print("noalloc non-finite stop", flush=True)
        rc_ref, ref, state_ref, hist_ref, _ = _doubling_run(lib, "rg_hip_exec_run", prog, win, wout, lout, 10, True)
        rc, got, state, hist, _ = _doubling_run(lib, "rg_hip_exec_run_noalloc", prog, win, wout, lout, 10, True)
        assert rc_ref == rc == 0
        # Step k records sum(w) = 1e38 * 2^(k+1): 2e38 after the first (finite), 4e38 > FLT_MAX
        # (inf) after the second, so the run stops there with two steps done.
        assert ref.nonfinite_step == got.nonfinite_step == 1 and ref.done == got.done == 2, (ref.done, got.done)
        assert np.array_equal(state.view(np.uint32), state_ref.view(np.uint32))
        assert np.array_equal(hist.view(np.uint64), hist_ref.view(np.uint64)) and np.isinf(hist[-1])
    finally:
        lib.rg_hip_program_free(prog)


def test_noalloc_failure_reports_the_steps_a_synchronization_confirmed():
    """An injected failure after 5 steps: with and without history, 5 steps done and the state
    after them (the final synchronization succeeded, so every launched step completed)."""
    lib = hip_abi()
    prog, (win,), (wout, lout) = _doubling_program(lib)
    try:
        for history in (False, True):
            print(f"noalloc injected failure, history={history}", flush=True)
            rc, res, state, _, failure = _doubling_run(lib, "rg_hip_exec_run_noalloc", prog, win, wout, lout, 10, history,
                                                       fail_after=5, x0=(1.0, 2.0, 3.0, 4.0))
            assert rc == -1 and failure == "injected failure" and res.done == 5, (history, res.done, failure)
            assert state.tolist() == [32.0, 64.0, 96.0, 128.0], (history, state)
    finally:
        lib.rg_hip_program_free(prog)


def test_run_descriptions_that_do_not_fit_the_program_are_refused_before_running():
    """Both run entries check every slot index, size and pointer of the description first."""
    lib = hip_abi()
    prog, (win,), (wout, lout) = _doubling_program(lib)
    err = ctypes.create_string_buffer(4096)
    try:
        for entry in ("rg_hip_exec_run", "rg_hip_exec_run_noalloc"):
            bad = {
                "slot out of range": dict(n_swaps=1, swaps=(ctypes.c_int64 * 2)(win, 1 << 40)),
                "swapped with itself": dict(n_swaps=1, swaps=(ctypes.c_int64 * 2)(win, win)),
                "copy beyond the slot": dict(n_copies=1, copies=(ctypes.c_int64 * 3)(win, wout, 5)),
                "history without buffer": dict(n_history=1, history_slots=(ctypes.c_int64 * 1)(lout)),
                "data beyond the slot": dict(n_data=1, data_slots=(ctypes.c_int64 * 1)(win), data_bytes=(ctypes.c_uint64 * 1)(17)),
            }
            for what, fields in bad.items():
                print(f"{entry}: {what}", flush=True)
                e = lib.rg_hip_exec_new(prog, err, len(err))
                assert e, err.value
                try:
                    d = RunDesc(steps=3, **fields)
                    res = RunResult()
                    assert getattr(lib, entry)(e, ctypes.byref(d), ctypes.byref(res)) == -1, what
                    assert res.done == 0, what
                    assert exec_failure(lib, e).startswith(entry + ":"), (what, exec_failure(lib, e))
                finally:
                    lib.rg_hip_exec_free(e)
    finally:
        lib.rg_hip_program_free(prog)
