"""Fused attention steps in device plans, on the CPU oracle.

The HIP planner replaces scaled, masked softmax attention and its reverse-mode subgraph by two
fused steps (RG_STEP_ATTN). The oracle executes those steps with the operations of the nodes
they replace, in the same order, so a device plan run on the oracle ("cpu_devplan") must give
the unfused CPU plan's results bit for bit. These tests check that the planner finds the regions
in the forms nn.MultiHeadAttention and the autodiff produce, leaves other programs alone, and
that the replacement is exact.
"""

import math

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import nn, random, workloads

from conftest import DEVPLAN


def _attention(q, k, v, mask=None, scale=True, fill=-1e9):
    s = q @ rg.swapaxes(k, -1, -2)
    if scale:
        s = s / math.sqrt(q.shape[-1])
    if mask is not None:
        s = rg.where(mask, s, fill)
    return nn.softmax(s) @ v


def _program(mask=None, scale=True, fill=-1e9):
    def loss(q, k, v, w):
        return (_attention(q, k, v, mask, scale, fill) * w).sum()
    return rg.value_and_grad(loss, argnums=(0, 1, 2))


def _inputs(shape, seed=0):
    r = np.random.default_rng(seed)
    return tuple(rg.tensor(r.normal(size=shape).astype(np.float32)) for _ in range(4))


def _steps(c):
    return [s for s in c._n.plan_summary() if s["kind"] == "attention"]


def _run_both(fn, args):
    dev = rg.compile(fn, args, device=DEVPLAN, validate="none")
    cpu = rg.compile(fn, args, device="cpu", validate="none")
    (v1, g1), (v2, g2) = dev(*args), cpu(*args)
    return dev, (v1, g1), (v2, g2)


def _assert_same(a, b):
    """Gradients bit for bit; the loss is a full sum, which device plans reduce in another order."""
    (v1, g1), (v2, g2) = a, b
    np.testing.assert_allclose(float(v1), float(v2), rtol=1e-4, atol=1e-4)  # a sum of ~1e4 terms of size ~1
    for x, y, name in zip(g1, g2, ("dq", "dk", "dv")):
        assert np.array_equal(x.numpy(), y.numpy()), f"{name}: max diff {np.abs(x.numpy() - y.numpy()).max()}"


@pytest.mark.parametrize("shape", [(2, 4, 64, 32), (3, 32, 16), (1, 2, 128, 64), (2, 1, 96, 16)])
def test_causal_attention_is_fused_and_exact(shape):
    t = shape[-2]
    fn = _program(mask=rg.tril(t))
    dev, a, b = _run_both(fn, _inputs(shape))
    steps = _steps(dev)
    assert [s["backward"] for s in steps] == [False, True], steps
    assert steps[0]["masked"] and steps[0]["tq"] == t and steps[0]["hd"] == shape[-1]
    _assert_same(a, b)


@pytest.mark.parametrize("scale,masked", [(False, False), (True, False), (False, True)])
def test_unscaled_and_unmasked_forms(scale, masked):
    shape = (2, 2, 64, 32)
    mask = rg.tril(64) if masked else None
    dev, a, b = _run_both(_program(mask=mask, scale=scale), _inputs(shape, 1))
    assert len(_steps(dev)) == 2
    _assert_same(a, b)


def test_masks_per_batch_and_fully_masked_rows():
    """A [B, 1, T, T] mask that varies per batch and hides every key of some query rows."""
    B, H, T, D = 2, 3, 64, 16
    m = np.tril(np.ones((B, 1, T, T), np.float32))
    m[1, 0, 5, :] = 0.0  # row 5 of batch 1 sees nothing: uniform weights
    m[0, 0, :, 40:] = 0.0
    dev, a, b = _run_both(_program(mask=rg.tensor(m)), _inputs((B, H, T, D), 2))
    steps = _steps(dev)
    assert len(steps) == 2 and steps[0]["masked"]
    _assert_same(a, b)


def test_forward_only_programs_fuse_the_forward():
    q, k, v, _ = _inputs((2, 2, 64, 32), 3)
    f = lambda q, k, v: _attention(q, k, v, rg.tril(64))
    dev = rg.compile(f, (q, k, v), device=DEVPLAN, validate="none")
    cpu = rg.compile(f, (q, k, v), device="cpu", validate="none")
    assert [s["backward"] for s in _steps(dev)] == [False]
    assert np.array_equal(dev(q, k, v).numpy(), cpu(q, k, v).numpy())


@pytest.mark.parametrize("shape", [(2, 2, 48, 32), (2, 2, 64, 24), (1, 1, 512, 16)])
def test_unsupported_sizes_keep_the_unfused_plan(shape):
    """Sequences that are not multiples of 32 or exceed 256, head sizes outside {16, 32, 64}."""
    fn = _program(mask=rg.tril(shape[-2]))
    dev, a, b = _run_both(fn, _inputs(shape, 4))
    assert _steps(dev) == []
    (v1, g1), (v2, g2) = a, b
    np.testing.assert_allclose(float(v1), float(v2), rtol=1e-4, atol=1e-4)


def test_intermediates_read_elsewhere_block_fusion():
    """The probabilities are also returned: the region is not closed, nothing is fused."""
    q, k, v, w = _inputs((2, 2, 64, 32), 5)

    def f(q, k, v):
        s = rg.where(rg.tril(64), q @ rg.swapaxes(k, -1, -2) / math.sqrt(32), -1e9)
        p = nn.softmax(s)
        return p @ v, p
    dev = rg.compile(f, (q, k, v), device=DEVPLAN, validate="none")
    assert _steps(dev) == []


def test_multi_head_attention_module_and_gpt_layers():
    """nn.MultiHeadAttention inside the GPT: one forward and one backward step per layer."""
    cfg = workloads.GPT_CONFIGS["C3"]._replace(batch=2, layers=2)
    step, state = workloads.gpt_train_step(cfg)
    dev = rg.compile(step, (state,), device=DEVPLAN, validate="none")
    kinds = [s["backward"] for s in _steps(dev)]
    assert kinds.count(False) == 2 and kinds.count(True) == 2, kinds
    # q, k and v are read in place from the projection that produced them, O is written with its
    # heads merged, and dq, dk, dv go straight into one gradient tensor: the transposes, slices
    # and pads around attention are gone.
    for s in _steps(dev):
        assert len(set(s["input_slots"][:3])) == 1, s
        if s["backward"]:
            assert len(set(s["output_slots"])) == 1, s
    ops = [s["op"] for s in dev._n.plan_summary() if s["kind"] == "instr"]
    assert "pad" not in ops and ops.count("transpose") <= 2, ops
    # Every layer reads the same causal mask: the first forward packs it, the rest reuse it.
    steps = _steps(dev)
    assert len({s["mask_bits_slot"] for s in steps}) == 1, steps
    assert [s["builds_mask_bits"] for s in steps].count(True) == 1
    assert steps[0]["builds_mask_bits"] and not steps[0]["backward"]
    cpu = rg.compile(step, (state,), device="cpu", validate="none")
    a = rg.run(dev, state, steps=2)
    b = rg.run(cpu, state, steps=2)
    np.testing.assert_allclose(a.history["aux"], b.history["aux"], rtol=1e-6)


def test_cpu_plans_never_fuse_attention():
    fn = _program(mask=rg.tril(64))
    c = rg.compile(fn, _inputs((2, 2, 64, 32)), device="cpu", validate="none")
    assert _steps(c) == []


@pytest.mark.parametrize("t", [32, 64, 128, 256])
def test_executed_share_of_causal_attention(t):
    """The engine's count of the 16 x 16 tiles the device kernels execute under a constant causal
    mask (the forward skips fully hidden tiles, the backward walks each wave's visible range):
    (n + 1) / 2n of them for n = t / 16 tiles per side, forward and backward; all without a mask."""
    shape = (2, 2, t, 32)
    n = t // 16
    for mask, want in ((rg.tril(t), (n + 1) / (2 * n)), (None, 1.0)):
        c = rg.compile(_program(mask=mask), _inputs(shape, 3), device=DEVPLAN, validate="none")
        steps = _steps(c)
        assert len(steps) == 2
        for s in steps:
            assert s["executed_flops"] == pytest.approx(want * s["flops"], rel=1e-12), (t, mask is None, s["backward"])
