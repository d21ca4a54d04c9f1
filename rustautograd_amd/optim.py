"""Optimizers as pairs of pure functions, traced into the compiled step like everything else.

`opt = adamw(3e-4)`; `state = opt.init(params)`; `params, state = opt.update(grads, state, params)`.
The state is a tree (a step counter plus per-parameter moments), so it lives in the run loop's
state next to the parameters. Each update is written with the arithmetic, in the order, of the
reference's python/rg/optim.py, so the same training run rounds the same way.
"""

import math
import typing

from . import tree
from .ops import cos, full, maximum, minimum, where, zeros_like


class Optimizer(typing.NamedTuple):
    init: typing.Callable    # params -> state
    update: typing.Callable  # (grads, state, params) -> (new params, new state)


# ---- learning-rate schedules: count -> rate ----

def constant(lr):
    return lambda count: lr


def cosine_decay(lr, total_steps, warmup_steps=0, min_lr=0.0):
    """A linear warm-up over `warmup_steps`, then half a cosine from `lr` down to `min_lr` at
    `total_steps`."""
    span = max(1, total_steps - warmup_steps)

    def rate(count):
        progress = minimum((count - warmup_steps) / span, 1.0)
        cosine = min_lr + (lr - min_lr) * 0.5 * (1.0 + cos(math.pi * maximum(progress, 0.0)))
        if warmup_steps == 0:
            return cosine
        return where(count >= warmup_steps, cosine, lr * (count + 1.0) / warmup_steps)

    return rate


def _as_schedule(lr):
    if callable(lr):
        return lr
    return constant(lr)


# ---- gradient transformations ----

def clip_by_global_norm(grads, max_norm):
    """`grads` scaled so that their joint L2 norm is at most `max_norm`."""
    total = tree.global_norm(grads)
    factor = max_norm / where(total >= max_norm, total, max_norm)
    return tree.map(lambda g: g * factor, grads)


def _prepare(grads, max_grad_norm):
    if not max_grad_norm:
        return grads
    return clip_by_global_norm(grads, max_grad_norm)


def _counter(params):
    """The step counter, a scalar of the parameters' dtype starting at 0."""
    return full((), 0, tree.leaves(params)[0].dtype)


def _zeros_like_tree(params):
    return tree.map(zeros_like, params)


# ---- optimizers ----

def sgd(lr, momentum=0.0, max_grad_norm=None):
    """Gradient descent, with heavy-ball momentum when `momentum` > 0."""
    schedule = _as_schedule(lr)

    def init(params):
        return {"count": _counter(params), "velocity": _zeros_like_tree(params)}

    def update(grads, state, params):
        grads = _prepare(grads, max_grad_norm)
        lr_now = schedule(state["count"])
        velocity = tree.map(lambda v, g: momentum * v + g, state["velocity"], grads) if momentum else state["velocity"]
        direction = velocity if momentum else grads
        new_params = tree.map(lambda p, d: p - lr_now * d, params, direction)
        return new_params, {"count": state["count"] + 1.0, "velocity": velocity}

    return Optimizer(init=init, update=update)


def rmsprop(lr, decay=0.9, eps=1e-8, max_grad_norm=None):
    """Steps scaled by a running average of squared gradients."""
    schedule = _as_schedule(lr)

    def init(params):
        return {"count": _counter(params), "square": _zeros_like_tree(params)}

    def update(grads, state, params):
        grads = _prepare(grads, max_grad_norm)
        lr_now = schedule(state["count"])
        square = tree.map(lambda s, g: decay * s + (1.0 - decay) * (g * g), state["square"], grads)
        new_params = tree.map(lambda p, g, s: p - lr_now * g / (s.sqrt() + eps), params, grads, square)
        return new_params, {"count": state["count"] + 1.0, "square": square}

    return Optimizer(init=init, update=update)


def adamw(lr, b1=0.9, b2=0.999, eps=1e-8, weight_decay=0.01, decay_filter=None, max_grad_norm=None):
    """Adam with decoupled weight decay. `decay_filter(param)` says which parameters decay; by
    default those with two or more dimensions (matrices), not biases or normalization scales."""
    schedule = _as_schedule(lr)
    decays = decay_filter if decay_filter is not None else (lambda param: param.ndim > 1)

    def init(params):
        return {"count": _counter(params), "mu": _zeros_like_tree(params), "nu": _zeros_like_tree(params)}

    def update(grads, state, params):
        grads = _prepare(grads, max_grad_norm)
        t = state["count"] + 1.0
        lr_now = schedule(state["count"])
        first = lambda m, g: b1 * m + (1.0 - b1) * g
        mu = tree.map(first, state["mu"], grads)
        nu = tree.map(lambda v, g: b2 * v + (1.0 - b2) * (g * g), state["nu"], grads)
        unbias1, unbias2 = 1.0 - b1 ** t, 1.0 - b2 ** t

        def apply_one(p, m, v):
            direction = (m / unbias1) / ((v / unbias2).sqrt() + eps)
            if weight_decay != 0.0 and decays(p):
                direction = direction + weight_decay * p
            return p - lr_now * direction

        return tree.map(apply_one, params, mu, nu), {"count": t, "mu": mu, "nu": nu}

    return Optimizer(init=init, update=update)


def adam(lr, b1=0.9, b2=0.999, eps=1e-8, max_grad_norm=None):
    """adamw without weight decay."""
    return adamw(lr, b1=b1, b2=b2, eps=eps, weight_decay=0.0, max_grad_norm=max_grad_norm)
