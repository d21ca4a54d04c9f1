"""Fused attention steps on the device, against the CPU oracle's unfused plan.

The device plan replaces scaled, masked softmax attention and its backward form by fused MFMA
kernels (score tiles in registers, softmax in base 2 with the scale folded into one operand).
Outputs and gradients are products and reductions: within 1e-4 of their own largest magnitude,
as for any matmul. The loss, a sum of attention outputs times random weights, cancels heavily, so
it is compared with the sum of the magnitudes it cancels, sum |O * w| (O from the oracle), at
1e-6: the size of the rounding any summation order leaves. Shapes cover every supported head size, ranks 3 and 4, causal and
per-batch masks with fully masked rows, and the C4 layer size.
"""

import math

import numpy as np
import pytest

import rustautograd_amd as rg

from helpers import close_rel
from test_attention_plan import _attention, _inputs, _program, _steps

pytestmark = pytest.mark.gpu


def _check(fn, args, what, mask=None, scale=True):
    hip = rg.compile(fn, args, device="hip", validate="none")
    cpu = rg.compile(fn, args, device="cpu", validate="none")
    assert [s["backward"] for s in _steps(hip)] == [False, True], _steps(hip)
    (v1, g1), (v2, g2) = hip(*args), cpu(*args)
    q, k, v, w = args
    out = rg.compile(lambda q, k, v: _attention(q, k, v, mask, scale), (q, k, v), device="cpu", validate="none")(q, k, v)
    magnitude = float(np.abs(out.numpy().astype(np.float64) * w.numpy()).sum())
    assert abs(float(v1) - float(v2)) <= 1e-6 * magnitude, (float(v1), float(v2), magnitude)
    for x, y, name in zip(g1, g2, ("dq", "dk", "dv")):
        close_rel(x.numpy(), y.numpy(), 1e-4, f"{what} {name}")


@pytest.mark.parametrize("shape", [(2, 4, 64, 32), (3, 32, 16), (1, 2, 128, 64), (2, 1, 96, 16), (4, 8, 256, 32), (2, 2, 256, 64)])
def test_causal_attention(shape):
    mask = rg.tril(shape[-2])
    _check(_program(mask=mask), _inputs(shape, sum(shape)), f"causal {shape}", mask)


@pytest.mark.parametrize("scale,masked", [(False, False), (True, False), (False, True)])
def test_unscaled_and_unmasked(scale, masked):
    shape = (2, 2, 128, 32)
    mask = rg.tril(128) if masked else None
    _check(_program(mask=mask, scale=scale), _inputs(shape, 7), f"scale={scale} masked={masked}", mask, scale)


def test_per_batch_masks_with_fully_masked_rows():
    B, H, T, D = 2, 3, 64, 16
    m = np.tril(np.ones((B, 1, T, T), np.float32))
    m[1, 0, 5, :] = 0.0
    m[0, 0, :, 40:] = 0.0
    _check(_program(mask=rg.tensor(m)), _inputs((B, H, T, D), 9), "per-batch mask", rg.tensor(m))


def test_forward_only():
    q, k, v, _ = _inputs((4, 8, 256, 32), 11)
    f = lambda q, k, v: nn_attention(q, k, v)
    hip = rg.compile(f, (q, k, v), device="hip", validate="none")
    cpu = rg.compile(f, (q, k, v), device="cpu", validate="none")
    assert [s["backward"] for s in _steps(hip)] == [False]
    close_rel(hip(q, k, v).numpy(), cpu(q, k, v).numpy(), 1e-4, "forward")


def nn_attention(q, k, v):
    from rustautograd_amd import nn
    s = rg.where(rg.tril(q.shape[-2]), q @ rg.swapaxes(k, -1, -2) / math.sqrt(q.shape[-1]), -1e9)
    return nn.softmax(s) @ v
