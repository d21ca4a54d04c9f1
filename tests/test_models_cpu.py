"""The Python surface and the BASELINE workloads on the CPU oracle, against torch float64.

torch (float64, autograd) is an independent library oracle for the model math that the
engine's plans execute: the GPT loss and every parameter gradient, activations, products of
every rank, and the optimizers. Restates the reference's tests/test_framework.py and
tests/test_api.py cases that touch the hot path, plus the run-loop semantics of
tests/engine.rs:663-745. Programs run on the CPU oracle (device "cpu") and, where noted, with
the HIP planner's plan on the oracle (device "cpu_devplan").
"""

import math

import numpy as np
import pytest
import torch

import rustautograd_amd as rg
from rustautograd_amd import nn, optim, random, workloads
from rustautograd_amd import tree as rtree

from conftest import DEVPLAN


def f64(x):
    return rg.tensor(np.asarray(x, dtype="float64"))


# ---- the language model (C3/C4 architecture) -------------------------------------------------

def torch_gpt_loss(p, x, y, heads, tied=False):
    """The same GPT written directly in torch against the same parameter values."""
    F = torch.nn.functional

    def ln(q, v):
        d = v - v.mean(-1, keepdim=True)
        return d / ((d * d).mean(-1, keepdim=True) + 1e-5).sqrt() * q["scale"] + q["shift"]

    t = x.shape[1]
    h = p["tok"]["table"][x] + p["pos"]["table"][torch.arange(t)]
    visible = torch.tril(torch.ones(t, t)) != 0
    for b in p["blocks"]:
        n = ln(b["norm1"], h)
        B, T, D = n.shape
        hd = D // heads
        qkv = (n @ b["attn"]["qkv"]["w"] + b["attn"]["qkv"]["b"]).reshape(B, T, 3, heads, hd).permute(2, 0, 3, 1, 4)
        s = qkv[0] @ qkv[1].transpose(-1, -2) / math.sqrt(hd)
        s = torch.where(visible, s, torch.tensor(-1e9, dtype=s.dtype))
        a = (torch.softmax(s, -1) @ qkv[2]).transpose(1, 2).reshape(B, T, D)
        h = h + a @ b["attn"]["out"]["w"] + b["attn"]["out"]["b"]
        z = ln(b["norm2"], h) @ b["fc1"]["w"] + b["fc1"]["b"]
        h = h + F.gelu(z, approximate="tanh") @ b["fc2"]["w"] + b["fc2"]["b"]
    hn = ln(p["norm"], h)
    logits = hn @ p["tok"]["table"].T if tied else hn @ p["head"]["w"]
    return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), y.reshape(-1))


def _tiny(tied, dtype="float64"):
    model = workloads.GPT(vocab=11, block=6, d=8, heads=2, layers=2, tied=tied)
    params = rtree.map(lambda v: v.cast(dtype), model.init(random.key(7)))
    return model, params


@pytest.mark.parametrize("tied", [False, True])
def test_gpt_loss_and_every_gradient_match_pytorch(tied):
    """test_framework.py:340-355: loss at rel 1e-11, every gradient at rtol 1e-8 (float64)."""
    model, params = _tiny(tied)
    r = np.random.default_rng(5)
    x = r.integers(0, 11, size=(3, 6)).astype("int32")
    y = r.integers(0, 11, size=(3, 6)).astype("int32")
    fn = rg.value_and_grad(lambda p, x, y: nn.cross_entropy(model(p, x), y))
    tp = rtree.map(lambda v: torch.tensor(v.numpy(), requires_grad=True), params)
    tv = torch_gpt_loss(tp, torch.tensor(x).long(), torch.tensor(y).long(), heads=2, tied=tied)
    tv.backward()
    want = [t.grad.numpy() for _, t in rtree.paths(tp)]
    for device in ("cpu", DEVPLAN):
        c = rg.compile(fn, (params, rg.tensor(x), rg.tensor(y)), device=device)
        assert c.report["status"] == "ok", c.report
        value, grads = c(params, rg.tensor(x), rg.tensor(y))
        assert float(value) == pytest.approx(tv.item(), rel=1e-11)
        got = rtree.paths(grads)
        assert len(got) == len(want)
        for (name, g), w in zip(got, want):
            np.testing.assert_allclose(g.numpy(), w, rtol=1e-8, atol=1e-10, err_msg=f"{device} {name}")


def test_gpt_train_step_matches_pytorch_for_three_steps():
    """The whole C3-style step (in-graph ids, AdamW) on the oracle against torch, float64."""
    cfg = workloads.GPTConfig(vocab=11, block=6, d=8, heads=2, layers=2, batch=3, tied=False, lr=1e-2)
    step, state = workloads.gpt_train_step(cfg)
    state = rtree.map(lambda v: v.cast("float64") if v.dtype == "float32" else v, state)
    c = rg.compile(step, (state,), device=DEVPLAN)
    out = rg.run(c, state, steps=3)
    # Replay the same ids in torch: the ids come from the key stream (random.randint).
    key = state["key"]
    tp = rtree.map(lambda v: torch.tensor(v.numpy(), requires_grad=True), state["params"])
    opt = torch.optim.AdamW([t for _, t in rtree.paths(tp)], lr=cfg.lr, weight_decay=0.0)
    losses = []
    for _ in range(3):
        k_next, k_ids = random.split(key)
        ids = random.randint(k_ids, (cfg.batch, cfg.block + 1), 0, cfg.vocab).numpy()
        key = k_next
        opt.zero_grad()
        loss = torch_gpt_loss(tp, torch.tensor(ids[:, :-1]).long(), torch.tensor(ids[:, 1:]).long(), heads=2)
        loss.backward()
        with torch.no_grad():
            # AdamW with decay only on ndim >= 2 parameters (python/rg/optim.py:378-390).
            for _, t in rtree.paths(tp):
                if t.ndim >= 2:
                    t.mul_(1 - cfg.lr * 0.01)
        opt.step()
        losses.append(loss.item())
    np.testing.assert_allclose(out.history["aux"], losses, rtol=1e-10)
    for (name, g), (_, t) in zip(rtree.paths(out.state["params"]), rtree.paths(tp)):
        np.testing.assert_allclose(g.numpy(), t.detach().numpy(), rtol=1e-8, atol=1e-11, err_msg=name)


# ---- products, activations, optimizers ---------------------------------------------------------

@pytest.mark.parametrize("sa,sb", [((3,), (3,)), ((2, 3), (3,)), ((3,), (3, 2)), ((2, 3), (3, 4)), ((5, 2, 3), (3, 4)),
                                   ((5, 2, 3), (5, 3, 4)), ((2, 3), (7, 3, 4)), ((1, 2, 3), (6, 3, 4)), ((5, 1, 2, 3), (1, 4, 3, 2))])
def test_matmul_ranks_match_numpy_and_torch_gradients(sa, sb):
    """test_framework.py:56-65."""
    r = np.random.default_rng(0)
    a, b = r.normal(size=sa), r.normal(size=sb)
    np.testing.assert_allclose((f64(a) @ f64(b)).numpy(), a @ b, rtol=1e-12)
    ga, gb = rg.grad(lambda p: ((p[0] @ p[1]) ** 2).sum())((f64(a), f64(b)))
    ta, tb = torch.tensor(a, requires_grad=True), torch.tensor(b, requires_grad=True)
    ((ta @ tb) ** 2).sum().backward()
    np.testing.assert_allclose(ga.numpy(), ta.grad.numpy(), rtol=1e-10)
    np.testing.assert_allclose(gb.numpy(), tb.grad.numpy(), rtol=1e-10)


def test_activations_and_losses_match_pytorch():
    """test_framework.py:103-123."""
    r = np.random.default_rng(3)
    x = f64(r.normal(size=(4, 5)))
    tx = torch.tensor(x.numpy())
    F = torch.nn.functional
    for mine, theirs in [(nn.softmax(x), F.softmax(tx, -1)), (nn.log_softmax(x), F.log_softmax(tx, -1)), (nn.relu(x), F.relu(tx)),
                         (nn.sigmoid(x), torch.sigmoid(tx)), (nn.softplus(x), F.softplus(tx)), (nn.silu(x), F.silu(tx))]:
        np.testing.assert_allclose(mine.numpy(), theirs.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(nn.gelu(x).numpy(), F.gelu(tx, approximate="tanh").numpy(), rtol=1e-12)
    labels = r.integers(0, 5, size=4)
    assert float(nn.cross_entropy(x, rg.tensor(labels))) == pytest.approx(F.cross_entropy(tx, torch.tensor(labels)).item(), rel=1e-12)
    t = f64(r.uniform(size=(4, 5)))
    assert float(nn.binary_cross_entropy_with_logits(x, t)) == pytest.approx(
        F.binary_cross_entropy_with_logits(tx, torch.tensor(t.numpy())).item(), rel=1e-12)
    np.testing.assert_allclose(nn.one_hot(rg.tensor([2, 0]), 3).numpy(), [[0, 0, 1], [1, 0, 0]])


def _trajectory(make_rg, make_torch, steps=40):
    r = np.random.default_rng(4)
    p0 = {"w": r.normal(size=(5, 3)), "b": r.normal(size=3)}
    x, y = r.normal(size=(16, 5)), r.normal(size=(16, 3))
    opt = make_rg()

    def step(s):
        v, g = rg.value_and_grad(lambda p: (((x @ p["w"] + p["b"]) - y) ** 2).mean())(s["p"])
        p, o = opt.update(g, s["o"], s["p"])
        return {"p": p, "o": o}, v

    p = {k: f64(v) for k, v in p0.items()}
    s0 = {"p": p, "o": opt.init(p)}
    out = rg.run(rg.compile(step, (s0,), device=DEVPLAN), s0, steps=steps)
    tp = {k: torch.tensor(v, requires_grad=True) for k, v in p0.items()}
    topt = make_torch(list(tp.values()))
    tx, ty = torch.tensor(x), torch.tensor(y)
    for _ in range(steps):
        topt.zero_grad()
        (((tx @ tp["w"] + tp["b"]) - ty) ** 2).mean().backward()
        topt.step()
    for k in p0:
        np.testing.assert_allclose(out.state["p"][k].numpy(), tp[k].detach().numpy(), rtol=1e-9, atol=1e-11)


def test_optimizers_follow_pytorch_exactly():
    """test_framework.py:157-164, with the HIP planner's plan."""
    _trajectory(lambda: optim.adam(0.01), lambda ps: torch.optim.Adam(ps, lr=0.01))
    _trajectory(lambda: optim.sgd(0.01), lambda ps: torch.optim.SGD(ps, lr=0.01))
    _trajectory(lambda: optim.sgd(0.01, momentum=0.9), lambda ps: torch.optim.SGD(ps, lr=0.01, momentum=0.9))
    _trajectory(lambda: optim.adamw(0.01, weight_decay=0.1, decay_filter=lambda p: True),
                lambda ps: torch.optim.AdamW(ps, lr=0.01, weight_decay=0.1))


# ---- BASELINE workloads at reduced size: the HIP planner's plan against the CPU plan -----------

def test_c1_linear_regression_converges():
    """README.md:233-247 / test_api.py:16-51: loss < 1e-3 and w close to true_w after 500 steps."""
    step, state, batch = workloads.linreg()
    c = rg.compile(step, (state, batch), device=DEVPLAN)
    out = rg.run(c, state, data=batch, steps=500)
    assert out.history["aux"][-1] < 1e-3
    np.testing.assert_allclose(out.state.numpy(), np.arange(8, dtype=np.float32), atol=1e-2)
    ref = rg.run(rg.compile(step, (state, batch), device="cpu"), state, data=batch, steps=500)
    np.testing.assert_allclose(out.history["aux"], ref.history["aux"], rtol=1e-4, atol=1e-7)


def test_c2_mlp_step_devplan_matches_cpu_plan():
    """The C2 program at batch 64 and width 128: device plan and CPU plan agree for 5 steps."""
    cfg = workloads.MLPConfig(batch=64, d_in=32, hidden=128, lr=1e-3)
    step, state = workloads.mlp_train_step(cfg)
    a = rg.run(rg.compile(step, (state,), device=DEVPLAN), state, steps=5)
    b = rg.run(rg.compile(step, (state,), device="cpu"), state, steps=5)
    np.testing.assert_allclose(a.history["aux"], b.history["aux"], rtol=1e-4)
    # Adam moves a parameter by about lr per step whatever the gradient's size, so an element
    # whose gradient is rounding noise may differ by a fraction of lr; a wrong gradient would
    # differ by ~lr * steps. Rows are reduced in a different order in the two plans.
    for (name, u), (_, v) in zip(rtree.paths(a.state["params"]), rtree.paths(b.state["params"])):
        np.testing.assert_allclose(u.numpy(), v.numpy(), rtol=1e-4, atol=0.01 * cfg.lr * 5, err_msg=name)


def test_c5_matrix_chain_stays_skinny_and_exact_enough():
    """C5 at n=256 with the device plan: the search runs, every product keeps a dimension of 8
    (no n x n x n product appears in the forward or backward chain), values match numpy in f64."""
    program, inputs = workloads.matrix_chain(n=256, k=8)
    c = rg.compile(program, inputs, device=DEVPLAN)
    assert c.report["graph"]["optimization"]["search"] is not None
    for s in c.plan_summary():
        if s.get("op", "").startswith("matmul"):
            a, b = s["arg_shapes"]
            k = a[0] if s["ta"] else a[-1]
            assert min(s["shape"][0], s["shape"][1], k) == 8, s
    value, gb, gc = c(*inputs)
    a, b, cc, d = (x.numpy().astype(np.float64) for x in inputs)
    chain = a @ b @ cc @ d
    # f32 accumulation over cancelling terms: bound the error by the size of the terms summed.
    assert abs(float(value) - chain.sum()) <= 1e-5 * np.abs(chain).sum()
    ones = np.ones((8, 8))
    np.testing.assert_allclose(gb.numpy(), a.T @ (ones @ (cc @ d).T), rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(gc.numpy(), (a @ b).T @ (ones @ d.T), rtol=1e-4, atol=1e-6)


# ---- the run loop (validate.rs:289-363) --------------------------------------------------------

def _gd(lr):
    def step(w, batch):
        x, y = batch
        loss = (w * x - y) ** 2 * 0.5
        g = rg.grad(lambda w: ((w * x - y) ** 2 * 0.5))(w)
        return w - g * lr, loss
    return step


def test_run_trains_and_stops_on_nonfinite_with_exact_replay():
    """engine.rs:681-702: converges to 3; a huge rate diverges and the run stops at the first
    non-finite step, which replay locates."""
    w0, batch = f64(0.0), (f64(2.0), f64(6.0))
    c = rg.compile(_gd(0.1), (w0, batch))
    out = rg.run(c, w0, data=batch, steps=200)
    assert out.steps == 200 and abs(float(out.state) - 3.0) < 1e-9 and out.history["aux"][-1] < 1e-15
    c = rg.compile(_gd(1000.0), (w0, batch))
    out = rg.run(c, w0, data=batch, steps=10_000)
    assert out.status == "stopped_nonfinite" and out.nonfinite_step is not None and out.nonfinite_step < 10_000
    info = rg.inspect(out)
    assert info["repro"]["step"] <= out.nonfinite_step


def test_run_matches_repeated_calls_exactly_and_cycles_batches():
    """engine.rs:704-717."""
    batches = [(f64(1.0), f64(2.0)), (f64(3.0), f64(1.0)), (f64(-2.0), f64(0.5))]
    for device in ("cpu", DEVPLAN):
        c = rg.compile(_gd(0.01), (f64(0.5), batches[0]), device=device)
        out = rg.run(c, f64(0.5), data=batches, steps=10)
        w = f64(0.5)
        for k in range(10):
            w, loss = c(w, batches[k % 3])
            assert float(loss) == out.history["aux"][k], k
        assert float(out.state) == float(w)


def test_run_handles_state_passthrough_and_swap_between_inputs():
    """engine.rs:719-730: new_a = b, new_b = a."""
    a, b = f64([1.0, 2.0]), f64([3.0, 4.0])
    c = rg.compile(lambda s: ((s[1], s[0]), s[0].sum()), ((a, b),), validate="basic")
    out = rg.run(c, (a, b), steps=3)
    assert out.state[0].tolist() == [3.0, 4.0] and out.state[1].tolist() == [1.0, 2.0]


def test_key_in_compiled_state_is_reproducible_and_advances():
    """test_framework.py:87-100."""
    def step(s):
        k1, k2 = random.split(s["key"])
        return {"key": k1, "x": s["x"] + random.normal(k2, (3,))}, s["x"].sum()

    s0 = {"key": random.key(1), "x": rg.zeros(3)}
    c = rg.compile(step, (s0,))
    a, b = rg.run(c, s0, steps=20), rg.run(c, s0, steps=20)
    assert a.state["x"].tolist() == b.state["x"].tolist()
    assert len(set(a.history["aux"])) == 20
    chunked = rg.run(c, s0, steps=20, callback=lambda r: None, every=7)
    assert chunked.state["x"].tolist() == a.state["x"].tolist()
    assert chunked.history["aux"] == a.history["aux"]


def test_run_with_iterator_callback_and_early_stop():
    """test_framework.py:220-243."""
    def step(w, b):
        return w + b, b.sum()

    w0 = rg.tensor([0.0])
    c = rg.compile(step, (w0, rg.tensor([1.0])))
    seen = []
    r = rg.run(c, w0, data=(rg.tensor([float(i)]) for i in range(10)), steps=100, callback=lambda r: seen.append(r.steps), every=4)
    assert r.status == "completed" and r.steps == 10 and seen == [4, 8, 10]
    assert r.state.tolist() == [45.0]
    assert r.history["aux"] == [float(i) for i in range(10)]
    r = rg.run(c, w0, data=rg.tensor([1.0]), steps=100, callback=lambda r: False if r.steps >= 6 else None, every=3)
    assert r.status == "stopped_by_callback" and r.steps == 6
    batches = [rg.tensor([1.0]), rg.tensor([2.0]), rg.tensor([4.0])]
    one = rg.run(c, w0, data=batches, steps=8)
    chunks = rg.run(c, w0, data=batches, steps=8, callback=lambda r: None, every=3)
    assert one.history == chunks.history
    with pytest.raises(rg.DiagnosticError) as e:
        rg.run(c, w0, data=iter([rg.tensor([1.0, 2.0])]), steps=1)
    assert e.value.diagnostic["code"] == "INPUT_SIGNATURE_MISMATCH"


def test_a_small_gpt_learns_a_pattern_and_its_sampler_continues_it():
    """examples/gpt.py of the reference end to end on the oracle: train on windows of a repeating
    text, then generate greedily (top_k=1) and with a nucleus filter (top_p=0.5)."""
    from rustautograd_amd import optim, workloads
    text = "abcd" * 100
    chars = sorted(set(text))
    tokens = rg.tensor(np.array([chars.index(c) for c in text], dtype=np.int32))
    model = workloads.GPT(vocab=4, block=4, d=16, heads=2, layers=1)
    params = model.init(random.key(0))
    opt = optim.adamw(5e-3, weight_decay=0.0)
    state = {"params": params, "opt": opt.init(params), "key": random.key(1)}
    step = workloads.window_train_step(model, opt, 8)
    r = rg.run(rg.compile(step, (state, tokens)), state, tokens, steps=200)
    assert r.history["aux"][-1] < 0.1 * r.history["aux"][0]
    for kw in ({"top_k": 1}, {"top_p": 0.5}):
        sampler = workloads.compile_sampler(model, r.state["params"], **kw)
        out = workloads.generate(sampler, 4, [0, 1, 2, 3], 8)
        assert "".join(chars[t] for t in out) == "abcdabcd", kw
