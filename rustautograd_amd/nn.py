"""Layers, activations, losses and initializers, built only on the public API.

A layer is a small stateless object: `layer.init(key)` returns its parameter tree and
`layer(params, x, ...)` applies it, so parameters are plain trees that differentiate, compile and
checkpoint like any other value. The parameter tree keys, the order in which `init` spends its
keys, and the arithmetic of every function (which fixes how results round) are those of the
reference's python/rg/nn.py; the code is this package's own.
"""

import math

from . import random
from .ops import (abs, argmax, argsort, concatenate, cumsum, equal, exp, eye, maximum, ones, stop_gradient, swapaxes,
                  take, take_along_axis, tanh, top_k, where, zeros)

_GELU_C = math.sqrt(2.0 / math.pi)
_MASKED = -1e9  # the score of a position a mask hides, and the logit of a filtered token


# ---- activations ----

def relu(x):
    return maximum(x, 0.0)


def sigmoid(x):
    return 1.0 / (1.0 + exp(-x))


def softplus(x):
    """log(1 + e^x), computed as max(x, 0) + log(1 + e^-|x|) so that it never overflows."""
    return maximum(x, 0.0) + (1.0 + exp(-abs(x))).log()


def silu(x):
    return x * sigmoid(x)


def gelu(x):
    """GELU with the tanh approximation: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    return 0.5 * x * (1.0 + tanh(_GELU_C * (x + 0.044715 * x * x * x)))


def _row_max(x, axis):
    # The shift that keeps exp() in range; it carries no gradient (the result does not depend on it).
    return stop_gradient(x.max(axis=axis, keepdims=True))


def logsumexp(x, axis=-1, keepdims=False):
    shift = _row_max(x, axis)
    total = exp(x - shift).sum(axis=axis, keepdims=True)
    lse = total.log() + shift
    return lse if keepdims else lse.squeeze(axis)


def log_softmax(x, axis=-1):
    normalizer = logsumexp(x, axis=axis, keepdims=True)
    return x - normalizer


def softmax(x, axis=-1):
    shifted = exp(x - _row_max(x, axis))
    return shifted / shifted.sum(axis=axis, keepdims=True)


def one_hot(idx, n, dtype="float32"):
    """Rows of the n x n identity picked by int32 `idx`."""
    identity = eye(n, dtype)
    return take(identity, idx, 0)


def dropout(key, x, rate, training=True):
    """Each element zeroed with probability `rate`, the rest scaled by 1 / (1 - rate)."""
    if rate == 0.0 or not training:
        return x
    survive = 1.0 - rate
    mask = random.bernoulli(key, survive, x.shape, x.dtype)
    return x * mask / survive


# ---- sampling filters: logits of tokens that must not be drawn become very negative ----

def top_k_logits(logits, k):
    """Keeps the `k` largest logits of the last axis (ties with the k-th are kept)."""
    kth = top_k(logits, k)[0][..., -1:]
    return where(logits >= kth, logits, _MASKED)


def top_p_logits(logits, p):
    """Nucleus filter: keeps the most probable tokens whose probabilities, summed in decreasing
    order, first reach `p` (the most probable token always stays)."""
    order = argsort(logits, descending=True)
    sorted_probs = softmax(take_along_axis(logits, order))
    mass_before = cumsum(sorted_probs) - sorted_probs
    keep_sorted = mass_before < p
    # Back from sorted positions to the original ones: the inverse permutation of `order`.
    inverse = argsort(order.cast(logits.dtype))
    return where(take_along_axis(keep_sorted, inverse), logits, _MASKED)


# ---- losses and metrics ----

def cross_entropy(logits, labels, axis=-1):
    """Mean negative log-likelihood of int32 `labels` under unnormalized `logits` (classes on the
    last axis)."""
    if axis != -1 and axis != logits.ndim - 1:
        raise ValueError(f"cross_entropy takes the classes on the last axis, not axis {axis}")
    log_probs = log_softmax(logits, axis)
    picked = take_along_axis(log_probs, labels.reshape(tuple(labels.shape) + (1,)))
    return -picked.mean()


def binary_cross_entropy_with_logits(logits, targets):
    per_element = maximum(logits, 0.0) - logits * targets + (1.0 + exp(-abs(logits))).log()
    return per_element.mean()


def mse_loss(pred, target):
    err = pred - target
    return (err * err).mean()


def l1_loss(pred, target):
    err = pred - target
    return abs(err).mean()


def accuracy(logits, labels):
    hits = equal(argmax(logits), labels)
    return hits.cast(logits.dtype).mean()


# ---- initializers: init(key, shape, dtype) ----

def normal_init(std=0.02):
    def init(key, shape, dtype="float32"):
        return random.normal(key, shape, dtype) * std
    return init


def _uniform_pm(key, shape, dtype, bound):
    return random.uniform(key, shape, dtype, low=-bound, high=bound)


def xavier_uniform(key, shape, dtype="float32"):
    return _uniform_pm(key, shape, dtype, math.sqrt(6.0 / (shape[-2] + shape[-1])))


def kaiming_uniform(key, shape, dtype="float32"):
    return _uniform_pm(key, shape, dtype, math.sqrt(6.0 / shape[-2]))


# ---- layers ----

class Layer:
    """Base of the layers here: `init(key)` builds the parameter tree, `__call__(params, ...)`
    applies it. Layers without parameters return an empty dict."""

    def init(self, key=None):
        return {}

    def __call__(self, params, *inputs):
        raise NotImplementedError


def _spend(key, n):
    """`n` keys split from `key`, in the order sub-layers receive them."""
    return random.split(key, n)


_DEFAULT_INIT = normal_init(0.02)


class Linear(Layer):
    """`x @ w + b` with `w` of shape (d_in, d_out): leading batch dimensions pass through."""

    def __init__(self, d_in, d_out, bias=True, init=None, dtype="float32"):
        self.d_in = d_in
        self.d_out = d_out
        self.bias = bias
        self.dtype = dtype
        self.w_init = _DEFAULT_INIT if init is None else init

    def init(self, key):
        params = {"w": self.w_init(key, (self.d_in, self.d_out), self.dtype)}
        if self.bias:
            params["b"] = zeros(self.d_out, self.dtype)
        return params

    def __call__(self, params, x):
        y = x @ params["w"]
        return y + params["b"] if self.bias else y


class Embedding(Layer):
    """int32 tokens to vectors: rows of `table`. The gradient accumulates into the rows used."""

    def __init__(self, n, d, init=None, dtype="float32"):
        self.n = n
        self.d = d
        self.dtype = dtype
        self.w_init = _DEFAULT_INIT if init is None else init

    def init(self, key):
        table = self.w_init(key, (self.n, self.d), self.dtype)
        return {"table": table}

    def __call__(self, params, idx):
        return take(params["table"], idx, 0)


class LayerNorm(Layer):
    """Normalizes the last axis to zero mean and unit variance, then scales and shifts."""

    def __init__(self, d, eps=1e-5, dtype="float32"):
        self.d = d
        self.eps = eps
        self.dtype = dtype

    def init(self, key=None):
        return dict(scale=ones(self.d, self.dtype), shift=zeros(self.d, self.dtype))

    def __call__(self, params, x):
        centred = x - x.mean(axis=-1, keepdims=True)
        variance = (centred * centred).mean(axis=-1, keepdims=True)
        return centred / (variance + self.eps).sqrt() * params["scale"] + params["shift"]


class MultiHeadAttention(Layer):
    """Self-attention over `heads` heads of `d // heads`. `mask` broadcasts to (T, T); nonzero
    means visible. With `key` and a dropout rate, the weights and the output are dropped out."""

    def __init__(self, d, heads, bias=True, dropout_rate=0.0, init=None, dtype="float32"):
        if d % heads != 0:
            raise ValueError(f"{heads} heads cannot split a model dimension of {d}")
        self.d = d
        self.heads = heads
        self.rate = dropout_rate
        self.qkv = Linear(d, 3 * d, bias, init, dtype)
        self.out = Linear(d, d, bias, init, dtype)

    def init(self, key):
        k_qkv, k_out = _spend(key, 2)
        return {"qkv": self.qkv.init(k_qkv), "out": self.out.init(k_out)}

    def __call__(self, params, x, mask=None, key=None):
        b, t, d = x.shape
        hd = d // self.heads
        # (b, t, 3d) -> (3, b, heads, t, hd): q, k and v for every head.
        qkv = self.qkv(params["qkv"], x).reshape(b, t, 3, self.heads, hd).transpose(2, 0, 3, 1, 4)
        q, k, v = qkv[0], qkv[1], qkv[2]
        scores = q @ swapaxes(k, -1, -2) / math.sqrt(hd)
        if mask is not None:
            scores = where(mask, scores, _MASKED)
        weights = softmax(scores)
        dropping = key is not None and self.rate > 0.0
        if dropping:
            k_weights, key = random.split(key)
            weights = dropout(k_weights, weights, self.rate)
        merged = (weights @ v).transpose(0, 2, 1, 3).reshape(b, t, d)
        out = self.out(params["out"], merged)
        return dropout(key, out, self.rate) if dropping else out


class TransformerBlock(Layer):
    """Pre-norm transformer block: x + attention(norm(x)), then x + mlp(norm(x)) with a GELU
    MLP of `mlp_ratio * d` hidden units."""

    def __init__(self, d, heads, mlp_ratio=4, dropout_rate=0.0, init=None, dtype="float32"):
        self.rate = dropout_rate
        self.norm1 = LayerNorm(d, dtype=dtype)
        self.norm2 = LayerNorm(d, dtype=dtype)
        self.attn = MultiHeadAttention(d, heads, True, dropout_rate, init, dtype)
        self.fc1 = Linear(d, mlp_ratio * d, True, init, dtype)
        self.fc2 = Linear(mlp_ratio * d, d, True, init, dtype)

    def init(self, key):
        k_attn, k_fc1, k_fc2 = _spend(key, 3)
        return {"norm1": self.norm1.init(), "attn": self.attn.init(k_attn), "norm2": self.norm2.init(),
                "fc1": self.fc1.init(k_fc1), "fc2": self.fc2.init(k_fc2)}

    def __call__(self, params, x, mask=None, key=None):
        k_attn, k_mlp = (None, None) if key is None else random.split(key)
        x = x + self.attn(params["attn"], self.norm1(params["norm1"], x), mask, k_attn)
        hidden = self.fc2(params["fc2"], gelu(self.fc1(params["fc1"], self.norm2(params["norm2"], x))))
        return x + (dropout(k_mlp, hidden, self.rate) if key is not None else hidden)


class GRUCell(Layer):
    """One step of a gated recurrent unit, h' = (1 - z) h + z c, with update gate z, reset
    gate r and candidate c = tanh(W_c [x, r h] + b_c). Unroll it in Python or step it with `scan`."""

    def __init__(self, d_in, d_hidden, init=None, dtype="float32"):
        self.d_hidden = d_hidden
        self.gates = Linear(d_in + d_hidden, 2 * d_hidden, True, init, dtype)
        self.cand = Linear(d_in + d_hidden, d_hidden, True, init, dtype)

    def init(self, key):
        k_gates, k_cand = _spend(key, 2)
        return {"gates": self.gates.init(k_gates), "cand": self.cand.init(k_cand)}

    def __call__(self, params, x, h):
        gate = sigmoid(self.gates(params["gates"], concatenate([x, h], -1)))
        update, reset = gate[..., :self.d_hidden], gate[..., self.d_hidden:]
        candidate = tanh(self.cand(params["cand"], concatenate([x, reset * h], -1)))
        return (1.0 - update) * h + update * candidate


class Sequential(Layer):
    """Layers applied in order. Plain functions (such as `gelu`) count as parameterless layers.
    Parameters are keyed by position: {"0": ..., "2": ...}."""

    def __init__(self, *layers):
        self.layers = layers

    def init(self, key):
        keys = _spend(key, max(1, len(self.layers)))
        return {str(i): layer.init(keys[i]) for i, layer in enumerate(self.layers) if hasattr(layer, "init")}

    def __call__(self, params, x):
        for i, layer in enumerate(self.layers):
            x = layer(params[str(i)], x) if hasattr(layer, "init") else layer(x)
        return x
