"""Counter-based random numbers with explicit keys.

A key is an int32 pair holding one 64-bit SplitMix64 state (high word first). Every draw is a
pure function of its key and its shape: the same key gives the same numbers on any device and
thread count, so a step that carries its key in the state can be replayed exactly. The engine's
`random_uniform`, `random_normal` and `key_split` operations do the bit work; the key packing and
the derived draws (integers, Bernoulli, Gumbel, categorical) are those of the reference's
python/rg/random.py.
"""

import numpy as np

from .ops import argmax, floor, log, maximum
from .tensor import apply, tensor

_GOLDEN_GAMMA = 0x9E3779B97F4A7C15  # the SplitMix64 increment


def key(seed):
    """The key for an integer seed: seed * gamma mod 2^64, as (high, low) int32 words."""
    state = (int(seed) * _GOLDEN_GAMMA) % (1 << 64)
    words = np.array([state >> 32, state & 0xFFFFFFFF], dtype=np.uint32).view(np.int32)
    return tensor(words, "int32")


def split(k, n=2):
    """`n` new independent keys as an (n, 2) tensor; unpacking it gives the keys."""
    return apply("key_split", k, n=n)


def _unit(k, shape, dtype):
    return apply("random_uniform", k, shape=list(shape), dtype=dtype)


def uniform(k, shape=(), dtype="float32", low=0.0, high=1.0):
    """Uniform values in [low, high)."""
    u = _unit(k, shape, dtype)
    if (low, high) == (0.0, 1.0):
        return u
    return low + (high - low) * u


def normal(k, shape=(), dtype="float32"):
    """Standard normal values (Box-Muller in float64, rounded to `dtype`)."""
    return apply("random_normal", k, shape=list(shape), dtype=dtype)


def randint(k, shape, low, high):
    """Uniform int32 values in [low, high). The draw is made in float64, so every integer of a
    range wider than 2^24 stays reachable."""
    u64 = _unit(k, shape, "float64")
    return floor(low + (high - low) * u64).cast("int32")


def bernoulli(k, p=0.5, shape=(), dtype="float32"):
    """1 with probability `p` and 0 otherwise, in `dtype`."""
    return apply("gt", tensor(float(p), dtype), _unit(k, shape, dtype))


def gumbel(k, shape=(), dtype="float32"):
    """Standard Gumbel values, -log(-log(u)) with u kept away from 0."""
    tiny = 1e-7 if dtype == "float32" else 1e-15
    return -log(-log(maximum(_unit(k, shape, dtype), tiny)))


def categorical(k, logits, axis=-1):
    """Indices drawn from the distribution softmax(logits) along `axis` (Gumbel-max)."""
    noise = gumbel(k, logits.shape, logits.dtype)
    return argmax(logits + noise, axis)
