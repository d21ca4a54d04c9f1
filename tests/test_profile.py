"""Profiles with a roofline: every operation row of `Compiled.profile` (the reference's
src/validate.rs:875-919 times operations) carries its algorithmic work, the rate it achieved and,
when the backend reports its device's peaks, the fraction of that peak.

The work of a step is priced two ways. Products (fused attention, and matrix products the
device runs on matrix cores) count their flops: 2 m n k per product. Every other step counts the
bytes it must move at least: each distinct input read once and each output written once, where
a row group's per-row values (last-axis reductions and what is computed from them alone) hold
one element per row and its reductions over the rows one per column. The expected figures below
are worked out by hand for each graph, so a dropped term, a double-counted input or a row value
counted at full size fails.

On the CPU the oracle runs the device-flavoured plans and reports no peaks; the HIP backend's
pure query of which products it streams is called through the C ABI without a device.
"""

import ctypes
import json
import os

import numpy as np
import pytest

import rustautograd_amd as rg

from conftest import DEVPLAN
from helpers import G
from test_attention_plan import _program

from rustautograd_amd import _native


def _profile(g, outs, inputs, device=DEVPLAN):
    c = g.compile(outs, inputs, device=device, optimize="standard")
    prof = json.loads(c.profile([rg.tensor(np.asarray(x))._t for x in inputs], 2))
    return c.plan_summary(), prof


def _row(prof, prefix):
    rows = [o for o in prof["operations"] if o["operation"].startswith(prefix)]
    assert len(rows) == 1, [o["operation"] for o in prof["operations"]]
    return rows[0]


def test_a_matrix_product_is_priced_by_its_flops():
    m, k, n = 64, 32, 48
    g = G()
    a, b = g.input((m, k), "float32"), g.input((k, n), "float32")
    steps, prof = _profile(g, [g.op("matmul", [a, b])], [np.ones((m, k), np.float32), np.ones((k, n), np.float32)])
    row = _row(prof, "matmul")
    assert row["bound"] == "mfma" and row["unit"] == "TFLOP/s"
    assert row["flops_per_run"] == 2 * m * n * k
    assert row["bytes_per_run"] == (m * k + k * n + m * n) * 4
    assert row["achieved"] > 0
    # The oracle reports no device peaks: no fraction is claimed.
    assert "unavailable" in prof["roofline"] and "fraction_of_peak" not in row
    assert [s["flops"] for s in steps] == [2 * m * n * k]


def test_a_batched_product_counts_every_problem():
    g = G()
    a, b = g.input((3, 16, 8), "float32"), g.input((3, 8, 24), "float32")
    steps, _ = _profile(g, [g.op("matmul", [a, b])], [np.ones((3, 16, 8), np.float32), np.ones((3, 8, 24), np.float32)])
    assert steps[0]["flops"] == 2 * 3 * 16 * 24 * 8 and steps[0]["bound"] == "mfma"


def test_a_fused_group_reads_each_distinct_input_once():
    shape = (128, 256)
    g = G()
    x = g.input(shape, "float32")
    y = g.bin("add", g.bin("mul", g.un("exp", x), x), g.scalar(1.0, "float32"))
    steps, prof = _profile(g, [y], [np.ones(shape, np.float32)])
    assert [s["kind"] for s in steps] == ["fused"], steps
    n = shape[0] * shape[1]
    # x is read by exp and by mul but moves once; the scalar constant is a splat of one element.
    assert steps[0]["bytes"] == (n + 1 + n) * 4 and steps[0]["bound"] == "hbm"
    row = _row(prof, "fused")
    assert row["bytes_per_run"] == steps[0]["bytes"] and row["unit"] == "GB/s"


def test_a_row_group_writes_per_row_values_once_per_row():
    rows, length = 96, 64
    g = G()
    x = g.input((rows, length), "float32")
    mx = g.op("max", [x], axes=[1], keepdims=True)
    e = g.un("exp", g.bin("sub", x, mx))
    s = g.op("sum", [e], axes=[1], keepdims=True)
    y = g.bin("div", e, s)
    steps, _ = _profile(g, [y, mx], [np.random.default_rng(0).normal(size=(rows, length)).astype(np.float32)])
    n = rows * length
    assert [(st["kind"], st["row_len"]) for st in steps] == [("fused", length), ("fused", 0)], steps
    # The row group: x in; exp(x - max) out in full, the row maxima and row sums out per row.
    assert steps[0]["bytes"] == (n + n + 2 * rows) * 4
    # The division: exp(x - max) and the row sums (a broadcast of one value per row) in, y out.
    assert steps[1]["bytes"] == (n + rows + n) * 4


def test_a_column_reduction_in_a_row_group_writes_one_value_per_column():
    rows, length = 80, 48
    g = G()
    x = g.input((rows, length), "float32")
    y = g.bin("mul", x, x)
    by_row = g.op("sum", [y], axes=[1], keepdims=True)
    by_col = g.op("sum", [y], axes=[0], keepdims=False)
    steps, _ = _profile(g, [by_row, by_col], [np.ones((rows, length), np.float32)])
    groups = [st for st in steps if st["kind"] == "fused" and st["row_len"]]
    assert len(groups) == 1 and groups[0]["column_reductions"] == 1, steps
    assert groups[0]["bytes"] == (rows * length + rows + length) * 4


def test_attention_counts_its_products_and_operands():
    bh_b, heads, t, hd = 2, 4, 64, 32
    r = np.random.default_rng(1)
    args = tuple(rg.tensor(r.normal(size=(bh_b, heads, t, hd)).astype(np.float32)) for _ in range(4))
    c = rg.compile(_program(mask=rg.tril(t)), args, device=DEVPLAN, validate="none")
    att = [s for s in c.plan_summary() if s["kind"] == "attention"]
    assert [s["backward"] for s in att] == [False, True]
    bh = bh_b * heads
    per_product = 2 * bh * t * t * hd
    assert att[0]["flops"] == 2 * per_product and att[1]["flops"] == 4 * per_product
    # Forward: q, k, v in and O out; backward: q, k, v, O, dO in and dq, dk, dv out.
    assert att[0]["bytes"] == 4 * bh * t * hd * 4 and att[1]["bytes"] == 8 * bh * t * hd * 4
    assert all(s["bound"] == "mfma" for s in att)
    prof = c.profile(*args, repeats=1)
    assert {o["bound"] for o in prof["operations"] if o["operation"].startswith("attention")} == {"mfma"}


def _hip():
    assert os.path.exists(_native.HIP_LIBRARY), "librg_hip.so is not built"
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    lib.rg_hip_gemm_streamed.restype = ctypes.c_int
    lib.rg_hip_gemm_streamed.argtypes = [ctypes.c_int32] + [ctypes.c_int64] * 4 + [ctypes.c_int32] * 2
    return lib


@pytest.mark.parametrize("m,n,k,batch,ta,tb,want", [
    (8, 4096, 4096, 1, 0, 0, 1),      # few rows, long K: the rows kernel
    (16, 1024, 2048, 1, 0, 1, 1),     # few rows against B^T: the dot kernel
    (4096, 1, 4096, 1, 0, 0, 1),      # a matrix-vector product
    (4096, 1, 4096, 1, 1, 0, 1),      # A^T x
    (4096, 4096, 8, 1, 0, 0, 1),      # a short-K outer product
    (16, 20, 8192, 1, 0, 0, 1),       # few outputs, long K: the tiny-output kernel
    (32, 64, 8192, 1, 0, 0, 0),       # both sides at least 32: matrix cores
    (1024, 1024, 1024, 1, 0, 0, 0),   # a square product: matrix cores
    (8, 4096, 4096, 2, 0, 0, 0),      # batched: matrix cores
    (16, 2048, 1000, 1, 0, 1, 0),     # B^T with K not a multiple of 256
])
def test_the_backend_says_which_products_it_streams(m, n, k, batch, ta, tb, want):
    assert _hip().rg_hip_gemm_streamed(0, m, n, k, batch, ta, tb) == want
    # float64 products never stream.
    assert _hip().rg_hip_gemm_streamed(1, m, n, k, batch, ta, tb) == 0


def test_without_a_device_the_backend_reports_no_peaks():
    lib = _hip()
    peaks = (ctypes.c_double * 3)()
    name = ctypes.create_string_buffer(256)
    lib.rg_hip_device_peaks.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.c_char_p, ctypes.c_size_t]
    if lib.rg_hip_available():
        pytest.skip("a device is visible")
    assert lib.rg_hip_device_peaks(peaks, name, 256) == 1 and name.value


@pytest.mark.gpu
def test_device_profile_reports_fractions_of_the_device_peaks():
    """On the GPU every row carries a fraction of MI355X's published peak (HBM 8 TB/s, fp32
    matrix cores 157.3 TFLOP/s): a streamed product against HBM, a square product against the
    matrix cores, an elementwise group against HBM. No fraction may exceed the peak."""
    r = np.random.default_rng(3)
    shapes = [(8, 2048), (2048, 2048), (512, 512), (512, 512)]
    vals = [r.normal(size=s).astype(np.float32) for s in shapes]
    g = G()
    a, b, c, d = (g.input(s, "float32") for s in shapes)
    outs = [g.op("matmul", [a, b]), g.op("matmul", [c, d]), g.un("exp", c)]
    steps, prof = _profile(g, outs, vals, device="hip")
    roof = prof["roofline"]
    assert "unavailable" not in roof, roof
    print("device:", roof["device"])
    assert roof["hbm_gb_per_s"] == 8000.0 and roof["fp32_tflop_per_s"] > 100
    assert 0 < roof["fraction_of_peak"] <= 1.0
    by_op = {o["operation"]: o for o in prof["operations"]}
    skinny = [o for k, o in by_op.items() if k.startswith("matmul [8, 2048]")]
    square = [o for k, o in by_op.items() if k.startswith("matmul [512, 512]")]
    assert len(skinny) == 1 and skinny[0]["bound"] == "hbm" and skinny[0]["peak"] == 8000.0
    assert len(square) == 1 and square[0]["bound"] == "mfma" and square[0]["peak"] == roof["fp32_tflop_per_s"]
    for o in prof["operations"]:
        print(f'{o["operation"]:40s} {o["achieved"]:10.2f} {o["unit"]:8s} {o["fraction_of_peak"]:.3f}')
        assert 0 < o["fraction_of_peak"] <= 1.0, o
