"""Random streams: the oracle against published SplitMix64 outputs and the golden fixture.

The fixture (tests/golden/rng_vectors.json) is written by tests/golden/make_rng_vectors.py, an
independent numpy-uint64 statement of SplitMix64 as rg applies it (src/plan.rs:1391-1435,
1532-1544; python/rg/random.py:10-14). The published first outputs of SplitMix64 seeded with 0
pin the mixing function and the counter layout without either restatement.
"""

import json
import os

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import random
from helpers import G

from conftest import DEVPLAN

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rng_vectors.json")

# SplitMix64 with state 0: the first four outputs (Vigna's splitmix64.c reference output).
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]


def _draw(key, op, device="cpu", **attrs):
    g = G()
    k = g.input((2,), "int32")
    out = g.op(op, [k], **attrs)
    return g.eval([out], [np.asarray(key, np.int32)], device=device)[0]


def test_uniform_of_key_zero_is_the_published_splitmix64_stream():
    for device in ("cpu", DEVPLAN):
        u64 = _draw([0, 0], "random_uniform", device, shape=[4], dtype="float64")
        assert u64.tolist() == [(v >> 11) * 2.0 ** -53 for v in SPLITMIX64_SEED0]
        u32 = _draw([0, 0], "random_uniform", device, shape=[4], dtype="float32")
        assert u32.tolist() == [float(np.float32((v >> 40) * 2.0 ** -24)) for v in SPLITMIX64_SEED0]


@pytest.fixture(scope="module")
def golden():
    with open(FIXTURE) as f:
        return json.load(f)


def test_streams_match_the_golden_vectors_bit_for_bit(golden):
    for case in golden["cases"]:
        k = case["key"]
        u32 = _draw(k, "random_uniform", shape=[64], dtype="float32")
        assert u32.tolist() == case["uniform_f32"], k
        u64 = _draw(k, "random_uniform", shape=[64], dtype="float64")
        assert [float(v).hex() for v in u64] == case["uniform_f64_hex"], k
        s = _draw(k, "key_split", n=4)
        assert s.dtype == np.int32 and s.tolist() == case["split4"], k


def test_normal_matches_the_golden_vectors_within_one_ulp(golden):
    """Box-Muller in f64 through libm; the fixture's numpy log/cos may differ by an ulp."""
    for case in golden["cases"]:
        k = case["key"]
        want = np.array([float.fromhex(h) for h in case["normal_f64_hex"]])
        got = _draw(k, "random_normal", shape=[32], dtype="float64")
        ulps = np.abs(got.view(np.int64) - want.view(np.int64))
        assert ulps.max() <= 2, (k, ulps.max())
        got32 = _draw(k, "random_normal", shape=[32], dtype="float32")
        want32 = np.array(case["normal_f32"], np.float32)
        assert np.abs(got32.view(np.int32).astype(np.int64) - want32.view(np.int32)).max() <= 1, k


def test_key_from_seed_matches_the_fixture(golden):
    for seed, want in golden["keys_from_seeds"].items():
        assert random.key(int(seed)).tolist() == want


def test_random_streams_are_deterministic_uniform_and_normal(oracle_threads):
    """engine.rs:845-868: statistical bounds, thread-count invariance, distinct keys."""
    g = G()
    k = g.input((2,), "int32")
    u = g.op("random_uniform", [k], shape=[100_000], dtype="float32")
    n = g.op("random_normal", [k], shape=[100_000], dtype="float64")
    ks = g.op("key_split", [k], n=3)
    c = g.compile([u, n, ks], [np.array([7, 11], np.int32)])
    key = [rg.tensor(np.array([7, 11], np.int32))._t]
    oracle_threads(1)
    serial = [rg.Tensor(t).numpy() for t in c.call(key)]
    oracle_threads(8)
    parallel = [rg.Tensor(t).numpy() for t in c.call(key)]
    assert all(np.array_equal(a, b) for a, b in zip(serial, parallel)), "stream must not depend on threads"
    us, ns = serial[0].astype(np.float64), serial[1]
    assert ((us >= 0) & (us < 1)).all()
    assert abs(us.mean() - 0.5) < 0.005 and abs(us.var() - 1 / 12) < 0.002
    assert abs(ns.mean()) < 0.02 and abs(ns.var() - 1) < 0.02
    assert abs((np.abs(ns) > 1.96).mean() - 0.05) < 0.003
    sp = serial[2].ravel()
    assert serial[2].shape == (3, 2) and sp[0] != sp[2] and sp[2] != sp[4]
    other = g.eval([u], [np.array([7, 12], np.int32)])[0]
    assert not np.array_equal(other, serial[0])


def test_random_is_pure_and_well_behaved():
    """test_framework.py:68-84 on the Python surface (eager ops run on the oracle here)."""
    k = random.key(42)
    assert random.normal(k, (4,)).tolist() == random.normal(k, (4,)).tolist()
    a, b = random.split(k)
    assert a.tolist() != b.tolist()
    assert random.split(k, 5).shape == (5, 2)
    ints = random.randint(k, (20000,), 3, 9).numpy()
    assert ints.dtype == np.int32 and ints.min() == 3 and ints.max() == 8
    assert abs(np.bincount(ints)[3:] / 20000 - 1 / 6).max() < 0.02
    u = random.uniform(k, (1000,), low=2.0, high=3.0).numpy()
    assert 2.0 <= u.min() and u.max() < 3.0
    with pytest.raises(rg.DiagnosticError) as e:
        random.normal(rg.tensor([1, 2, 3]), (2,))
    assert e.value.diagnostic["code"] == "INVALID_KEY"
