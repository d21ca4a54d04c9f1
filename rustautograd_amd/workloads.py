"""The five benchmark programs, written against the public API.

C1 linear regression, C2 MLP regression, C3/C4 char-level GPT training steps, C5 matrix chain.
The GPT follows the reference's examples/gpt.py:20-68 (tok/pos embeddings, pre-norm transformer
blocks, final LayerNorm, head, cross-entropy, AdamW) with the batch of token ids drawn inside the
step from a key carried in the state, so a run never returns to the host.
"""

import math
from typing import NamedTuple

import numpy as np

import rustautograd_amd as rg
from rustautograd_amd import nn, optim, random


# ---- C1: linear regression (README example of the reference) ---------------------------------

def linreg(n=256, d=8, lr=0.05, seed=0):
    """Returns (step, w0, batch): `w -= lr * grad(mean((X@w - y)^2))`, loss as aux."""
    x = np.random.default_rng(seed).normal(size=(n, d)).astype(np.float32)
    y = x @ np.arange(d, dtype=np.float32)

    def loss(w, x, y):
        r = x @ w - y
        return (r * r).mean()

    def step(w, batch):
        xb, yb = batch
        l, g = rg.value_and_grad(loss)(w, xb, yb)
        return w - lr * g, l

    return step, rg.zeros(d), (rg.tensor(x), rg.tensor(y))


# ---- C2: MLP regression ---------------------------------------------------------------------

class MLPConfig(NamedTuple):
    batch: int = 4096
    d_in: int = 512
    hidden: int = 2048
    lr: float = 1e-3
    weight_decay: float = 0.01


def mlp_train_step(cfg=MLPConfig()):
    """Linear(512->2048)-gelu-Linear(2048->2048)-gelu-Linear(2048->1), AdamW; x ~ N(0,1) drawn in
    the step from the state key, target = sum(sin(x[:, :16]), axis=1, keepdims)."""
    model = nn.Sequential(nn.Linear(cfg.d_in, cfg.hidden), nn.gelu, nn.Linear(cfg.hidden, cfg.hidden), nn.gelu, nn.Linear(cfg.hidden, 1))
    params = model.init(random.key(0))
    opt = optim.adamw(cfg.lr, weight_decay=cfg.weight_decay)

    def loss_fn(p, x, t):
        return nn.mse_loss(model(p, x), t)

    def step(state):
        k_next, k_x = random.split(state["key"])
        x = random.normal(k_x, (cfg.batch, cfg.d_in))
        target = rg.sin(x[:, :16]).sum(axis=1, keepdims=True)
        value, grads = rg.value_and_grad(loss_fn)(state["params"], x, target)
        p, o = opt.update(grads, state["opt"], state["params"])
        return {"params": p, "opt": o, "key": k_next}, value

    return step, dict(params=params, opt=opt.init(params), key=random.key(1))


# ---- C3 / C4: character-level GPT -------------------------------------------------------------

class GPTConfig(NamedTuple):
    vocab: int
    block: int
    d: int
    heads: int
    layers: int
    batch: int
    tied: bool = False
    lr: float = 3e-4


GPT_CONFIGS = {
    "C3": GPTConfig(vocab=96, block=128, d=128, heads=4, layers=4, batch=32, tied=True),
    "C4": GPTConfig(vocab=96, block=256, d=256, heads=8, layers=6, batch=32, tied=False),
}


class GPT:
    """The character-level GPT of the reference's examples/gpt.py:20-47: token and position
    embeddings, pre-norm transformer blocks under a causal mask, a final layer norm and a linear
    head (read from the token table when `tied`). `init` spends split keys in the example's
    order: token table, position table, head, then one key per block."""

    def __init__(self, vocab, block, d=128, heads=4, layers=4, tied=False):
        self.block, self.tied = block, tied
        self.layers = {
            "tok": nn.Embedding(vocab, d),
            "pos": nn.Embedding(block, d),
            "norm": nn.LayerNorm(d),
            "head": nn.Linear(d, vocab, bias=False),
        }
        self.stack = [nn.TransformerBlock(d, heads) for _ in range(layers)]
        self.causal = rg.tril(block)

    def init(self, key):
        k_tok, k_pos, k_head, *k_blocks = random.split(key, len(self.stack) + 3)
        params = {"tok": self.layers["tok"].init(k_tok), "pos": self.layers["pos"].init(k_pos), "norm": self.layers["norm"].init(),
                  "blocks": [blk.init(kb) for blk, kb in zip(self.stack, k_blocks)]}
        if not self.tied:
            params["head"] = self.layers["head"].init(k_head)
        return params

    def __call__(self, params, idx):
        length = idx.shape[1]
        h = self.layers["tok"](params["tok"], idx) + self.layers["pos"](params["pos"], rg.arange(length))
        visible = self.causal[:length, :length]
        for blk, p_blk in zip(self.stack, params["blocks"]):
            h = blk(p_blk, h, visible)
        h = self.layers["norm"](params["norm"], h)
        if self.tied:
            return h @ params["tok"]["table"].T
        return self.layers["head"](params["head"], h)


def gpt_train_step(cfg):
    """Returns (step, state). Each step draws `batch` sequences of `block + 1` ids uniform in
    [0, vocab) from the state key (random.randint: f64 uniform, floor, int32), trains on
    x = ids[:, :-1], y = ids[:, 1:] with cross-entropy and AdamW, and returns the loss as aux."""
    model = GPT(cfg.vocab, cfg.block, cfg.d, cfg.heads, cfg.layers, cfg.tied)
    params = model.init(random.key(0))
    opt = optim.adamw(cfg.lr, weight_decay=0.01)

    def loss_fn(p, x, y):
        return nn.cross_entropy(model(p, x), y)

    def step(state):
        k_next, k_ids = random.split(state["key"])
        ids = random.randint(k_ids, (cfg.batch, cfg.block + 1), 0, cfg.vocab)
        x, y = ids[:, :-1], ids[:, 1:]
        value, grads = rg.value_and_grad(loss_fn)(state["params"], x, y)
        p, o = opt.update(grads, state["opt"], state["params"])
        return {"params": p, "opt": o, "key": k_next}, value

    return step, dict(params=params, opt=opt.init(params), key=random.key(1))


def gpt_gemm_flops(cfg):
    """2*M*N*K summed over every product of one training step (forward, both backward products
    of each forward product); the algorithmic flop count of the step."""
    b, t, d, h, f, v = cfg.batch, cfg.block, cfg.d, cfg.heads, 4 * cfg.d, cfg.vocab
    hd = d // h
    tokens = b * t
    per_layer = tokens * d * 3 * d + b * h * t * hd * t + b * h * t * t * hd + tokens * d * d + tokens * d * f + tokens * f * d
    fwd = cfg.layers * per_layer + tokens * d * v
    return 2 * 3 * fwd


# ---- C5: matrix chain -------------------------------------------------------------------------

def matrix_chain(n=4096, k=8, seed=0):
    """sum((A@B)@C@D) with A (k,n), B and C (n,n), D (n,k), all ~ N(0, 1/sqrt(n)); gradients with
    respect to B and C. Written in the expensive left-to-right order."""
    rng = np.random.default_rng(seed)
    sigma = 1.0 / math.sqrt(n)
    a, b, c, d = (rng.normal(0.0, sigma, size=s).astype(np.float32) for s in ((k, n), (n, n), (n, n), (n, k)))

    def f(a, b, c, d):
        return (((a @ b) @ c) @ d).sum()

    def program(a, b, c, d):
        value, (gb, gc) = rg.value_and_grad(f, argnums=(1, 2))(a, b, c, d)
        return value, gb, gc

    return program, tuple(rg.tensor(x) for x in (a, b, c, d))


# ---- generation: the inference-side caller of the same run loop --------------------------------

def windows(tokens, key, batch, block):
    """`batch` random windows of `block + 1` consecutive tokens: inputs and next-token targets
    (the reference's examples/gpt.py:50-55), drawn on the device from `key`."""
    n = tokens.shape[0]
    start = random.randint(key, (batch,), 0, n - block - 1)
    w = rg.take(tokens, start[:, None] + rg.arange(block + 1))
    return w[:, :-1], w[:, 1:]


def window_train_step(model, opt, batch):
    """A training step over random windows of a token tensor passed as data: `step(state, tokens)`."""

    def loss_fn(params, x, y):
        return nn.cross_entropy(model(params, x), y)

    def step(state, tokens):
        k_next, k_win, _ = random.split(state["key"], 3)
        x, y = windows(tokens, k_win, batch, model.block)
        value, grads = rg.value_and_grad(loss_fn)(state["params"], x, y)
        params, opt_state = opt.update(grads, state["opt"], state["params"])
        return {"params": params, "opt": opt_state, "key": k_next}, value

    return step


def compile_sampler(model, params, temperature=1.0, top_k=None, top_p=None, device=None):
    """A compiled step that appends one sampled token to a fixed-length context (the reference's
    examples/gpt.py:71-86): the model's last-position logits, scaled by 1/temperature, optionally
    filtered to the top k or the nucleus p, drawn by the Gumbel-max trick; the context shifts left
    by one. `rg.run(sampler, state, steps=n)` then generates n tokens with no Python per token."""

    def step(state):
        k_next, k_draw = random.split(state["key"])
        logits = model(params, state["ctx"])[:, -1, :] / temperature
        if top_k:
            logits = nn.top_k_logits(logits, top_k)
        if top_p:
            logits = nn.top_p_logits(logits, top_p)
        token = random.categorical(k_draw, logits)
        ctx = rg.concatenate([state["ctx"][:, 1:], token[:, None]], axis=1)
        return {"ctx": ctx, "key": k_next}, token[0]

    start = {"ctx": rg.zeros((1, model.block), "int32"), "key": random.key(0)}
    return rg.compile(step, (start,), validate="basic", device=device)


def generate(sampler, block, prompt_ids, n, seed=0):
    """`n` token ids continuing `prompt_ids`. The context is fixed at `block` ids: the prompt is
    left-padded with its first id (or cut to its last `block` ids)."""
    ids = ([prompt_ids[0]] * block + list(prompt_ids))[-block:]
    state = {"ctx": rg.tensor([ids], "int32"), "key": random.key(seed)}
    out = rg.run(sampler, state, steps=n)
    return [int(t) for t in out.history["aux"]]
