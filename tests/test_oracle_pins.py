"""Closed-form pins for the oracle's casts, wrapping int32 arithmetic and f32 libm calls.

These hold the CPU oracle (oracle/cpu_exec.cpp) to values fixed outside it:
- casts follow Rust `as` (reference src/plan.rs:1624-1642): float to int truncates toward zero,
  saturates at the i32 bounds and maps NaN to 0; float64 to float32 rounds once, to nearest even;
- int32 add, sub and mul wrap modulo 2^32 (src/plan.rs:1272-1287, `wrapping_add/sub/mul`); the
  expected values here come from Python's unbounded integers reduced modulo 2^32;
- f32 transcendentals are glibc's f32 routines, element by element (src/tensor.rs:215-227 calls
  `f32::exp` and friends, which Rust lowers to libm's `expf`, `logf`, ...). The expected bits here
  come from calling those routines directly through ctypes.
A wrong rounding mode, a dropped saturation, an f64 detour in the f32 math or a widened integer
fails one of them.
"""

import ctypes
import ctypes.util
import struct

import numpy as np
import pytest

from conftest import DEVPLAN
from helpers import op, run_graph, t

DEVICES = ["cpu", DEVPLAN]
I32_MIN, I32_MAX = -2 ** 31, 2 ** 31 - 1


def wrap32(v):
    v &= 0xFFFFFFFF
    return v - 2 ** 32 if v >= 2 ** 31 else v


@pytest.mark.parametrize("device", DEVICES)
def test_float_to_int_casts_truncate_saturate_and_zero_nan(device):
    f32_in = [np.nan, 3e9, -3e9, 2.9, -2.9, -0.0, np.inf, -np.inf, 2147483520.0, -2147483648.0, 0.99999994, -1.5]
    f32_want = [0, I32_MAX, I32_MIN, 2, -2, 0, I32_MAX, I32_MIN, 2147483520, I32_MIN, 0, -1]
    f64_in = [np.nan, 2147483647.5, 2147483648.0, -2147483648.9, -2147483649.0, 1e300, -1e300, 7.999999999, -7.999999999]
    f64_want = [0, I32_MAX, I32_MAX, I32_MIN, I32_MIN, I32_MAX, I32_MIN, 7, -7]
    for values, dtype, want in ((f32_in, "float32", f32_want), (f64_in, "float64", f64_want)):
        got = run_graph(device, lambda g, i: op(g, "cast", [i[0]], dtype="int32"), [t(values, dtype)])[0]
        assert got.dtype == np.int32
        assert got.tolist() == want, (dtype, got.tolist())


def _f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


@pytest.mark.parametrize("device", DEVICES)
def test_float64_to_float32_rounds_once_to_nearest_even(device):
    # Each expected value is written as its bit pattern, worked out by hand from the binary
    # expansion of the input: no float conversion of this test's own is trusted.
    cases = [
        (1e300, 0x7F800000),                  # overflow: +inf
        (-1e300, 0xFF800000),                 # -inf
        (1e-50, 0x00000000),                  # below half the smallest subnormal: +0
        (-1e-50, 0x80000000),                 # -0
        (1.0000001, 0x3F800001),              # 1 + 1.0e-7 lies nearer 1 + 2^-23 than 1
        (1.0 + 2.0 ** -24, 0x3F800000),       # a tie: rounds to even (1.0)
        (1.0 + 3 * 2.0 ** -24, 0x3F800002),   # a tie: rounds to even (1 + 2^-22)
        (2.0 ** -149, 0x00000001),            # smallest subnormal
        (2.0 ** -150, 0x00000000),            # half of it, a tie to even: 0
        (3 * 2.0 ** -150, 0x00000002),        # 1.5 subnormal steps, tie to even: 2 steps
        (16777217.0, 0x4B800000),             # 2^24 + 1: tie to even, 2^24
        (3.4028234663852886e38, 0x7F7FFFFF),  # the largest float32 (2^128 - 2^104), exact
        (3.4028235677973366e38, 0x7F800000),  # 2^128 - 2^103, the midpoint to 2^128: tie to even overflows
        (3.4028235677973362e38, 0x7F7FFFFF),  # one f64 step below that midpoint: the largest float32
    ]
    x = t([c[0] for c in cases], "float64")
    got = run_graph(device, lambda g, i: op(g, "cast", [i[0]], dtype="float32"), [x])[0]
    assert [_f32_bits(v) for v in got.tolist()] == [c[1] for c in cases]


@pytest.mark.parametrize("device", DEVICES)
def test_int32_to_float_casts_round_to_nearest_even(device):
    ints = [16777217, 16777219, I32_MAX, I32_MIN, -16777217, 0, 1]
    got = run_graph(device, lambda g, i: op(g, "cast", [i[0]], dtype="float32"), [t(ints, "int32")])[0]
    # 2^24+1 and 2^24+3 are ties: to even gives 2^24 and 2^24+4; 2^31-1 rounds up to 2^31.
    assert got.tolist() == [16777216.0, 16777220.0, 2147483648.0, -2147483648.0, -16777216.0, 0.0, 1.0]
    got64 = run_graph(device, lambda g, i: op(g, "cast", [i[0]], dtype="float64"), [t(ints, "int32")])[0]
    assert got64.tolist() == [float(v) for v in ints]


INT_PAIRS = [
    (I32_MAX, 1), (I32_MIN, -1), (65536, 65536), (46341, 46341), (I32_MIN, I32_MIN), (I32_MAX, I32_MAX),
    (I32_MIN, 1), (-1, I32_MIN), (0, I32_MIN), (123456789, -987654321), (-7, 3), (I32_MAX, I32_MIN),
]
INT_RULES = {
    "add": lambda a, b: wrap32(a + b),
    "sub": lambda a, b: wrap32(a - b),
    "mul": lambda a, b: wrap32(a * b),
    "gt": lambda a, b: int(a > b),
    "ge": lambda a, b: int(a >= b),
}


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("name", sorted(INT_RULES))
def test_int32_arithmetic_wraps_and_compares_at_the_bounds(device, name):
    a = t([p[0] for p in INT_PAIRS], "int32")
    b = t([p[1] for p in INT_PAIRS], "int32")
    got = run_graph(device, lambda g, i: op(g, name, [i[0], i[1]]), [a, b])[0]
    assert got.dtype == np.int32
    assert got.tolist() == [INT_RULES[name](x, y) for x, y in INT_PAIRS]
    # Broadcast modes (scalar on either side, and a row) take the same wrapping path.
    s = t(I32_MAX, "int32")
    got = run_graph(device, lambda g, i: op(g, name, [i[0], i[1]]), [s, b])[0]
    assert got.tolist() == [INT_RULES[name](I32_MAX, y) for _, y in INT_PAIRS]
    got = run_graph(device, lambda g, i: op(g, name, [i[0], i[1]]), [a, s])[0]
    assert got.tolist() == [INT_RULES[name](x, I32_MAX) for x, _ in INT_PAIRS]


def _libm():
    return ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")


def _libm_f32(name, *cols):
    fn = getattr(_libm(), name)
    fn.restype = ctypes.c_float
    fn.argtypes = [ctypes.c_float] * len(cols)
    return np.array([fn(*vals) for vals in zip(*[c.tolist() for c in cols])], dtype=np.float32)


def _sweep(lo, hi, n, seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([np.linspace(lo, hi, n // 2), rng.uniform(lo, hi, n - n // 2)]).astype(np.float32)


# The last group of each sweep holds inputs where glibc's f32 routine and the correctly rounded
# value (f64 routine, then one rounding to f32) differ: an oracle that computed in f64 and
# rounded would fail there.
F32_UNARY = {
    "exp": ("expf", [_sweep(-104.0, 89.0, 3000, 1), np.float32([-87.33655, 88.72283, 88.72284, -103.97208, 1e-8, -1e-8]),
                     np.float32([74.87860107421875, 38.80278778076172, 63.36878204345703, 64.13075256347656])]),
    "log": ("logf", [_sweep(1e-6, 1e6, 2000, 2), np.float32([1e-45, 1e-40, 1.17549435e-38, 3.4028235e38, 1.0, 0.99999994]),
                     np.float32([169350.171875, 568367.8125, 637039.125, 797303.5])]),
    "sin": ("sinf", [_sweep(-1e4, 1e4, 2000, 3), np.float32([1e5, -1e6, 3.4e38, 1e-30, 3.1415927, 1e4 + 0.5]),
                     np.float32([6492.89111328125, -8969.9658203125, 2330.833740234375, 5061.3212890625])]),
    "cos": ("cosf", [_sweep(-1e4, 1e4, 2000, 4), np.float32([1e5, -1e6, 3.4e38, 1e-30, 1.5707964, 1e4 + 0.5]),
                     np.float32([5741.04150390625, 4295.5751953125, -1802.2213134765625, -2715.783935546875])]),
    "tanh": ("tanhf", [_sweep(-12.0, 12.0, 2000, 5), np.float32([-10.0, 10.0, 9.01, -9.01, 1e-20, 0.55]),
                       np.float32([0.20494461059570312, 0.5177186131477356, -0.6730678081512451, 0.4529299736022949])]),
}


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("name", sorted(F32_UNARY))
def test_f32_transcendentals_are_glibc_f32_bit_for_bit(device, name):
    fname, parts = F32_UNARY[name]
    x = np.concatenate(parts)
    want = _libm_f32(fname, x)
    got = run_graph(device, lambda g, i: op(g, name, [i[0]]), [t(x)])[0]
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


@pytest.mark.parametrize("device", DEVICES)
def test_f32_pow_is_glibc_powf_bit_for_bit(device):
    rng = np.random.default_rng(6)
    # The last four pairs are ones where powf and the correctly rounded power differ.
    base = np.concatenate([rng.uniform(0.0, 4.0, 1500), rng.uniform(-3.0, 0.0, 300).round(), np.float32([2.0, 10.0, 0.5, -2.0, 1.0001]),
                           np.float32([2.231518268585205, 0.3359132409095764, 0.9762961268424988, 3.137620449066162])])
    expo = np.concatenate([rng.uniform(-40.0, 40.0, 1500), rng.integers(-9, 10, 300).astype(np.float64), np.float32([127.0, 38.0, 149.0, 127.0, 80000.0]),
                           np.float32([-32.935428619384766, -26.017990112304688, 37.92976379394531, 5.070365905761719])])
    base, expo = base.astype(np.float32), expo.astype(np.float32)
    want = _libm_f32("powf", base, expo)
    got = run_graph(device, lambda g, i: op(g, "pow", [i[0], i[1]]), [t(base), t(expo)])[0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("device", DEVICES)
def test_f32_math_inside_fused_groups_is_the_same_libm_call(device):
    """A fused chain evaluates each op with the same f32 routine as the single instruction."""
    x = _sweep(-8.0, 8.0, 4096, 7)
    got = run_graph(device, lambda g, i: op(g, "tanh", [op(g, "exp", [op(g, "neg", [i[0]])])]), [t(x)])[0]
    want = _libm_f32("tanhf", _libm_f32("expf", -x))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
