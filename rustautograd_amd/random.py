"""Explicit, splittable random numbers: every function is pure in its key.

Keys are int32 pairs; streams are SplitMix64 of (key, index), so the same key gives the same
numbers on every device and thread count (reference python/rg/random.py, src/plan.rs:1391-1435).
"""

from ._core import _op, argmax, floor, log, maximum, tensor

_GAMMA = 0x9E3779B97F4A7C15


def key(seed):
    """A key from an integer seed: seed * GAMMA mod 2**64, split into signed hi and lo words."""
    mixed = seed * _GAMMA % (1 << 64)
    signed = lambda v: v - (1 << 32) if v >= (1 << 31) else v
    return tensor([signed(mixed >> 32), signed(mixed & 0xFFFFFFFF)], "int32")


def split(k, n=2):
    """`n` independent keys, as a tensor of shape (n, 2) that unpacks into keys."""
    return _op("key_split", k, n=n)


def uniform(k, shape=(), dtype="float32", low=0.0, high=1.0):
    """Uniform floats in [low, high)."""
    u = _op("random_uniform", k, shape=list(shape), dtype=dtype)
    return u if low == 0.0 and high == 1.0 else low + (high - low) * u


def normal(k, shape=(), dtype="float32"):
    """Standard normal floats (Box-Muller in float64, then rounded to `dtype`)."""
    return _op("random_normal", k, shape=list(shape), dtype=dtype)


def randint(k, shape, low, high):
    """Uniform int32 in [low, high). Drawn in float64 so every integer of a wide range is reachable."""
    u = _op("random_uniform", k, shape=list(shape), dtype="float64")
    return floor(low + (high - low) * u).cast("int32")


def bernoulli(k, p=0.5, shape=(), dtype="float32"):
    """1 with probability `p`, else 0, as floats."""
    return _op("gt", tensor(float(p), dtype), _op("random_uniform", k, shape=list(shape), dtype=dtype))


def gumbel(k, shape=(), dtype="float32"):
    u = _op("random_uniform", k, shape=list(shape), dtype=dtype)
    eps = 1e-7 if dtype == "float32" else 1e-15
    return -log(-log(maximum(u, eps)))


def categorical(k, logits, axis=-1):
    """Indices sampled from unnormalized log-probabilities with the Gumbel-max trick."""
    return argmax(logits + gumbel(k, logits.shape, logits.dtype), axis)
