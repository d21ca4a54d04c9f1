"""rustautograd_amd: rg's trace / differentiate / compile / validate / run pipeline with an
MI355X-native HIP execution backend.

    import rustautograd_amd as rg
    step = rg.compile(train_step, (state, data), device="hip")
    result = rg.run(step, state, data, steps=300)

The engine (graph, autodiff, optimizer, planner, run loop) is C++ (`_rg`); every plan step runs
as a hand-written CDNA4 kernel in librg_hip.so. The public names are those of the reference's
python/rg/__init__.py.
"""

from ._native import DiagnosticError
from .tensor import Tensor, Tracer, Value, tensor
from .ops import (
    abs, arange, argmax, argsort, broadcast_to, clip, concatenate, cos, cumsum, equal, exp, expand_dims, eye, flip, floor, full,
    linspace, log, matmul, max, maximum, mean, min, minimum, not_equal, ones, ones_like, reshape, sign, sin, sort, sqrt, square,
    squeeze, stack, std, stop_gradient, sum, swapaxes, take, take_along_axis, tanh, top_k, transpose, tril, var, where, zeros,
    zeros_like,
)
from .transforms import custom_vjp, grad, hessian, jvp, value_and_grad
from .control import cond, scan, while_loop
from .program import Compiled, Report, RunResult, compile, devices, inspect, run
from .checkpoint import load, save
from . import nn, optim, random, tree

__version__ = "0.2.0"
