"""Writes rng_vectors.json: SplitMix64 streams of rg's random ops, computed with numpy uint64.

The algorithm is the published SplitMix64 (Steele, Lea and Flood, "Fast splittable
pseudorandom number generators", OOPSLA 2014; constants as in Vigna's splitmix64.c), applied
the way the reference's src/plan.rs:1391-1435 and 1532-1544 apply it:

  key      = (u32(k[0]) << 32) | u32(k[1])                   (read_key, plan.rs:1411-1414)
  uniform  = (mix(key + (j+1)*GAMMA) >> (64 - mantissa)) * 2^-mantissa, mantissa 24 or 53
  normal   = sqrt(-2 ln(1 - u(2j+1))) * cos(2 pi u(2j+2)),  u(c) = (mix(key + c*GAMMA) >> 11) * 2^-53
  split[j] = mix(key + (j+1)*GAMMA_SPLIT) as (hi, lo) int32 pairs   (key_split, plan.rs:1416-1425)
  key(seed)= seed * GAMMA mod 2^64 as (hi, lo) int32                 (python/rg/random.py:10-14)

Run from the repository root: python tests/golden/make_rng_vectors.py
"""

import json
import os

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
GAMMA_SPLIT = np.uint64(0xD1B54A32D192ED03)


def mix(z):
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def key_bits(k):
    return np.uint64((int(k[0]) & 0xFFFFFFFF) << 32 | (int(k[1]) & 0xFFFFFFFF))


def stream(key, counters, gamma=GAMMA):
    with np.errstate(over="ignore"):
        return mix(key + np.asarray(counters, dtype=np.uint64) * gamma)


def uniform(k, n, mantissa):
    bits = stream(key_bits(k), np.arange(1, n + 1))
    return (bits >> np.uint64(64 - mantissa)).astype(np.float64) * 0.5 ** mantissa


def normal(k, n):
    j = np.arange(n, dtype=np.uint64)
    unit = lambda c: (stream(key_bits(k), c) >> np.uint64(11)).astype(np.float64) * 0.5 ** 53
    u1, u2 = 1.0 - unit(2 * j + 1), unit(2 * j + 2)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2 * np.pi * u2)


def split(k, n):
    bits = stream(key_bits(k), np.arange(1, n + 1), GAMMA_SPLIT)
    hi = (bits >> np.uint64(32)).astype(np.uint32).view(np.int32)
    lo = (bits & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.int32)
    return np.stack([hi, lo], axis=1)


def key(seed):
    mixed = (seed * 0x9E3779B97F4A7C15) % (1 << 64)
    to_i32 = lambda v: v - (1 << 32) if v >= (1 << 31) else v
    return [to_i32(mixed >> 32), to_i32(mixed & 0xFFFFFFFF)]


def main():
    keys = [[0, 0], [7, 11], [7, 12], [-1, -2], [2147483647, -2147483648]] + [key(s) for s in (0, 1, 42)]
    cases = []
    for k in keys:
        cases.append({
            "key": k,
            "uniform_f32": [float(v) for v in uniform(k, 64, 24).astype(np.float32)],
            "uniform_f64_hex": [float(v).hex() for v in uniform(k, 64, 53)],
            "normal_f64_hex": [float(v).hex() for v in normal(k, 32)],
            "normal_f32": [float(v) for v in normal(k, 32).astype(np.float32)],
            "split4": split(k, 4).tolist(),
        })
    out = {"source": "tests/golden/make_rng_vectors.py", "keys_from_seeds": {str(s): key(s) for s in (0, 1, 42, 12345)}, "cases": cases}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rng_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
