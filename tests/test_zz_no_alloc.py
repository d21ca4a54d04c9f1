"""rg_hip_exec_run_noalloc, the run loop that allocates nothing, against rg_hip_exec_run.

Two calls in a row through the C ABI, the second with smaller inputs: a gradient-descent program
with cycled batches, per-step history and buffer swaps, then a smaller one whose state is handed
back by copies. Each must give rg_hip_exec_run's state and history bit for bit. A run whose
buffers exceed the static scratch is refused before anything runs.
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
