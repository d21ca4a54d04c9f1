"""Kernels that compute several plan steps: elementwise groups computed in the epilogue of the
product they read, against the same program with every group in its own kernel
(RG_HIP_EPILOGUE=0); column sums of such a group's output computed in the same kernel, against
the reduction kernel (RG_HIP_EPILOGUE_SUMS=0); and independent products launched as one kernel,
against single launches (RG_HIP_PAIR=0).

The combined kernel applies the group's operations, in the group's order, to the product's
finished outputs (the values the product's own kernel would have stored), so the two programs
must agree bit for bit: the state after one C4 step and after a device loop of C2, every loss on
the way. `step_runs_in` names the pairs. C4 has twelve: each layer's GELU forward, computed by
the first MLP product, which also stores its own output for the backward pass, and each layer's
GELU backward, computed by the product that forms the activation gradient (five at the
product's step, the last layer's at its own, since the weight-gradient product between them
reads the slot the group writes). C2 has one by default (its first layer's activation: the only
product of at least 1024 tiles) and four with RG_HIP_EPILOGUE=all, among them a weight gradient
that runs its parameter's whole AdamW update in its epilogue.
"""

import numpy as np
import pytest

import rustautograd_amd as rg
from rustautograd_amd import _pytree, workloads

pytestmark = pytest.mark.gpu


def _pairs(compiled):
    runs_in = compiled._n.step_runs_in()
    return [(k, r) for k, r in enumerate(runs_in) if r != k]


def _bits(tree):
    return [np.atleast_1d(np.asarray(x.numpy())).view(np.uint8) for x in _pytree.leaves(tree)]


@pytest.mark.parametrize("name,mode,steps,pairs", [("C4", None, 1, 12), ("C2", None, 5, 1), ("C2", "all", 5, 4)])
def test_products_with_epilogues_match_separate_kernels_bit_for_bit(monkeypatch, name, mode, steps, pairs):
    step, state = workloads.mlp_train_step() if name == "C2" else workloads.gpt_train_step(workloads.GPT_CONFIGS[name])
    print(f"{name}: compile with and without product epilogues ({mode or 'default'}), {steps} device steps", flush=True)
    monkeypatch.setenv("RG_HIP_PAIR", "0")  # pairs of products: a test below
    monkeypatch.setenv("RG_HIP_EPILOGUE_SUMS", "0")  # column sums in the epilogue: a test below
    monkeypatch.setenv("RG_HIP_EPILOGUE", "0")
    plain = rg.compile(step, (state,), validate="none", device="hip")
    if mode:
        monkeypatch.setenv("RG_HIP_EPILOGUE", mode)
    else:
        monkeypatch.delenv("RG_HIP_EPILOGUE")
    fused = rg.compile(step, (state,), validate="none", device="hip")
    assert _pairs(plain) == [] and len(_pairs(fused)) == pairs, _pairs(fused)
    r0 = rg.run(plain, state, steps=steps)
    r1 = rg.run(fused, state, steps=steps)
    assert r0.status == r1.status == "completed"
    assert np.array_equal(np.array(r0.history["aux"]).view(np.uint64), np.array(r1.history["aux"]).view(np.uint64))
    for a, b in zip(_bits(r0.state), _bits(r1.state)):
        assert np.array_equal(a, b)


def test_products_launched_together_match_single_launches_bit_for_bit(monkeypatch):
    """Each C4 layer's fc1 input-gradient and weight-gradient products are independent, adjacent
    and on the same tile shape: they run as one kernel (its blocks split between them, each
    running the single product's tile code), at the first one's step, and in five of the six
    layers the fc2 weight gradient a few steps earlier joins them (in the last layer's backward
    pass it reads a slot the GELU backward group between them overwrites, so it stays). The
    attention projection's weight gradient moves down to run with the q, k, v projection's
    (both on 64x64 tiles). The state after a step and the loss equal the single launches' bit
    for bit (RG_HIP_PAIR=0)."""
    step, state = workloads.gpt_train_step(workloads.GPT_CONFIGS["C4"])
    print("C4: compile with and without paired product launches, 1 device step", flush=True)
    monkeypatch.setenv("RG_HIP_PAIR", "0")
    single = rg.compile(step, (state,), validate="none", device="hip")
    monkeypatch.delenv("RG_HIP_PAIR")
    paired = rg.compile(step, (state,), validate="none", device="hip")
    plan = paired.plan_summary()

    def product_pairs(compiled):
        return [(k, r) for k, r in _pairs(compiled) if plan[k].get("op", "").startswith("matmul") and plan[r].get("op", "").startswith("matmul")]
    grouped = product_pairs(paired)
    assert product_pairs(single) == [] and len(grouped) == 17 and len({r for _, r in grouped}) == 12, grouped
    r0 = rg.run(single, state, steps=1)
    r1 = rg.run(paired, state, steps=1)
    assert r0.status == r1.status == "completed"
    assert np.array_equal(np.array(r0.history["aux"]).view(np.uint64), np.array(r1.history["aux"]).view(np.uint64))
    for a, b in zip(_bits(r0.state), _bits(r1.state)):
        assert np.array_equal(a, b)


def test_streamed_products_launched_together_match_single_launches_bit_for_bit(monkeypatch):
    """C5's chain ((8 x 4096) x 4096 x 4096 and its gradients) streams its products through the
    row, dot and outer-product kernels. The forward product x W1 and the outer product of the
    gradient run as one launch; the second forward product, the dot product that forms the
    gradient of x W1 and the outer product that forms W2's gradient as another; and the last
    forward product (8 x 8 outputs over K = 4096) with the outer product that forms W1's gradient
    as a third. Each block runs its own product's block code (the 8-wave reduction of the last
    forward product by 4 waves that each run two waves' lanes), so the results are the single
    launches' bit for bit."""
    program, inputs = workloads.matrix_chain()
    print("C5: compile with and without grouped streamed products", flush=True)
    monkeypatch.setenv("RG_HIP_PAIR", "0")
    single = rg.compile(program, inputs, device="hip", validate="none")
    monkeypatch.delenv("RG_HIP_PAIR")
    grouped = rg.compile(program, inputs, device="hip", validate="none")
    assert _pairs(single) == [] and _pairs(grouped) == [(1, 0), (3, 2), (4, 2), (6, 5)], _pairs(grouped)
    for a, b in zip(single(*inputs), grouped(*inputs)):
        assert np.array_equal(np.asarray(a.numpy()).view(np.uint32), np.asarray(b.numpy()).view(np.uint32))


def test_column_sums_in_their_producers_match_the_reduction_kernel(monkeypatch):
    """Each C4 layer's two bias gradients that are column sums of a kernel's output are computed by
    that kernel: the fc1 bias gradient by the product whose epilogue computes the GELU backward
    (each lane sums its rows in registers, the tile's lanes and waves combine in a fixed order,
    one partial row per 128-row tile), the q, k, v bias gradient by the attention backward (one
    partial row per batch element); the fold area's partial rows are then folded in order. The
    sums' order differs from the reduction kernel's (RG_HIP_EPILOGUE_SUMS=0), so after one step
    the bias leaves (the biases and their AdamW moments) agree to rounding, within 1e-4 of each
    leaf's largest value (7e-7 measured on MI355X), and every other leaf and the loss bit for bit.
    The key third of the q, k, v bias is left out: its true gradient is exactly zero (softmax is
    invariant to a per-row constant), so AdamW normalises rounding noise of either order to the
    learning rate's size."""
    step, state = workloads.gpt_train_step(workloads.GPT_CONFIGS["C4"])
    print("C4: compile with and without column sums in their producers, 1 device step", flush=True)
    monkeypatch.setenv("RG_HIP_EPILOGUE_SUMS", "0")
    plain = rg.compile(step, (state,), validate="none", device="hip")
    monkeypatch.delenv("RG_HIP_EPILOGUE_SUMS")
    fused = rg.compile(step, (state,), validate="none", device="hip")
    plan = fused.plan_summary()
    absorbed = [(k, r) for k, r in enumerate(fused._n.step_runs_in()) if r != k and plan[k].get("op") == "sum"]
    assert len(absorbed) == 12 and not [k for k, r in enumerate(plain._n.step_runs_in()) if r != k and plan[k].get("op") == "sum"]
    assert sum(plan[r]["kind"] == "attention" for _, r in absorbed) == 6
    r0 = rg.run(plain, state, steps=1)
    r1 = rg.run(fused, state, steps=1)
    assert r0.status == r1.status == "completed" and r0.history["aux"] == r1.history["aux"]
    differing = 0
    for a, b in zip(_pytree.leaves(r0.state), _pytree.leaves(r1.state)):
        a, b = np.asarray(a.numpy()), np.asarray(b.numpy())
        if np.array_equal(np.atleast_1d(a).view(np.uint8), np.atleast_1d(b).view(np.uint8)):
            continue
        differing += 1
        assert a.shape in ((1024,), (768,)), a.shape
        scale = max(float(np.abs(a).max()), 1e-30)
        keep = np.ones(a.shape, bool)
        if a.shape == (768,):
            keep[256:512] = False
        assert float(np.abs(a.astype(np.float64) - b)[keep].max()) <= 1e-4 * scale
    assert 0 < differing <= 36, differing
