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

    def batch(key):
        x = random.normal(key, (cfg.batch, cfg.d_in))
        return x, rg.sin(x[:, :16]).sum(axis=1, keepdims=True)

    def loss_and_grads(state):
        _, k_x = random.split(state["key"])
        return rg.value_and_grad(loss_fn)(state["params"], *batch(k_x))

    def step(state):
        k_next, k_x = random.split(state["key"])
        value, grads = rg.value_and_grad(loss_fn)(state["params"], *batch(k_x))
        p, o = opt.update(grads, state["opt"], state["params"])
        return {"params": p, "opt": o, "key": k_next}, value

    _describe(step, loss_and_grads, cfg.lr, cfg.weight_decay)
    return step, dict(params=params, opt=opt.init(params), key=random.key(1))


def _describe(step, loss_and_grads, lr, weight_decay):
    """Attaches to a training step the program of its first half, `loss_and_grads(state) ->
    (loss, gradient tree)` with the same draws, and its AdamW settings, for tests that compare
    a step's gradients and updates on their own."""
    step.loss_and_grads = loss_and_grads
    step.adamw = {"lr": lr, "weight_decay": weight_decay, "b1": 0.9, "b2": 0.999, "eps": 1e-8}


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

    def batch(key):
        ids = random.randint(key, (cfg.batch, cfg.block + 1), 0, cfg.vocab)
        return ids[:, :-1], ids[:, 1:]

    def loss_and_grads(state):
        _, k_ids = random.split(state["key"])
        return rg.value_and_grad(loss_fn)(state["params"], *batch(k_ids))

    def step(state):
        k_next, k_ids = random.split(state["key"])
        value, grads = rg.value_and_grad(loss_fn)(state["params"], *batch(k_ids))
        p, o = opt.update(grads, state["opt"], state["params"])
        return {"params": p, "opt": o, "key": k_next}, value

    _describe(step, loss_and_grads, cfg.lr, 0.01)
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


# ---- token streams and generation: callers of the same run loop -------------------------------

class TokenWindows:
    """Training windows cut from one long 1-D token tensor inside the compiled step.

    A draw picks `batch` start offsets uniformly in [0, n - block - 1) (`random.randint`) and
    gathers the `block + 1` consecutive ids at each: the first `block` are the inputs, the same
    span shifted by one the next-token targets. The reference draws its windows this way
    (examples/gpt.py:50-55); its published GPT losses (benches/results_gpt.json) depend on it."""

    def __init__(self, batch, block):
        self.batch, self.block = batch, block

    def positions(self, starts):
        """[batch, block + 1] token positions: every start plus 0, 1, ..., block."""
        return starts.reshape(self.batch, 1) + rg.arange(self.block + 1)

    def __call__(self, tokens, key):
        last_start = tokens.shape[0] - self.block - 1
        span = rg.take(tokens, self.positions(random.randint(key, (self.batch,), 0, last_start)))
        return span[:, :self.block], span[:, 1:]


def windows(tokens, key, batch, block):
    """(inputs, targets) of one `TokenWindows(batch, block)` draw."""
    return TokenWindows(batch, block)(tokens, key)


def window_train_step(model, opt, batch):
    """`step(state, tokens)`: one optimizer step on a fresh draw of windows from `tokens`, the
    token tensor `rg.run` passes as data. The state key is split three ways, as the reference's
    training step does (examples/gpt.py:58-68): the key carried to the next step, the window
    draw's key, and the model's dropout key, which this dropout-free GPT does not spend."""
    draw = TokenWindows(batch, model.block)
    loss_and_grads = rg.value_and_grad(lambda params, inputs, targets: nn.cross_entropy(model(params, inputs), targets))

    def step(state, tokens):
        carried, for_windows, _for_dropout = random.split(state["key"], 3)
        loss, grads = loss_and_grads(state["params"], *draw(tokens, for_windows))
        new_params, new_opt = opt.update(grads, state["opt"], state["params"])
        return {"params": new_params, "opt": new_opt, "key": carried}, loss

    return step


def prompt_state(prompt_ids, block, seed=0):
    """A sampler state for a prompt: the context holds the prompt's last `block` ids, left-padded
    with its first id when it is shorter, and the key is `random.key(seed)`."""
    ids = list(prompt_ids)[-block:]
    ids = [ids[0]] * (block - len(ids)) + ids
    return {"ctx": rg.tensor([ids], "int32"), "key": random.key(seed)}


class Sampler:
    """Autoregressive generation as a compiled one-token step.

    The state is a fixed-length context of ids and a key. A step scores the context, divides the
    logits of its last position by `temperature`, applies the optional top-k and nucleus
    filters, draws one id by the Gumbel-max trick (`random.categorical`) and slides the context
    left by one position to append the id, which is also the step's aux output. `rg.run(...,
    steps=n)` thus generates n ids with no Python between them. Behaviour of the reference's
    examples/gpt.py:71-93."""

    def __init__(self, model, params, temperature=1.0, top_k=None, top_p=None, device=None):
        self.model, self.params, self.block, self.temperature = model, params, model.block, temperature
        self.filters = []
        if top_k:
            self.filters.append(lambda z: nn.top_k_logits(z, top_k))
        if top_p:
            self.filters.append(lambda z: nn.top_p_logits(z, top_p))
        self.program = rg.compile(self.advance, (prompt_state([0], self.block),), validate="basic", device=device)

    def next_logits(self, context):
        scores = self.model(self.params, context)[:, -1, :] / self.temperature
        for keep in self.filters:
            scores = keep(scores)
        return scores

    def advance(self, state):
        carried, for_draw = random.split(state["key"])
        picked = random.categorical(for_draw, self.next_logits(state["ctx"]))
        shifted = rg.concatenate([state["ctx"][:, 1:], picked.reshape(1, 1)], axis=1)
        return {"ctx": shifted, "key": carried}, picked[0]

    def generate(self, prompt_ids, n, seed=0):
        """`n` ids continuing `prompt_ids`, one device step each."""
        return generate(self.program, self.block, prompt_ids, n, seed)


def compile_sampler(model, params, temperature=1.0, top_k=None, top_p=None, device=None):
    """The compiled one-token step of a `Sampler` (what `generate` runs)."""
    return Sampler(model, params, temperature, top_k, top_p, device).program


def generate(sampler, block, prompt_ids, n, seed=0):
    """`n` ids continuing `prompt_ids` from a compiled sampler step over a `block`-id context."""
    out = rg.run(sampler, prompt_state(prompt_ids, block, seed), steps=n)
    return [int(t) for t in out.history["aux"]]
