"""The nanoGPT-shaped model, synthetic text and batches of the 1,000-step
loss-curve comparison (tests/test_gpu_loss_curve.py and
tests/loss_curve_floor.py).

The model follows the reference's benchmark configuration
(benchmarks/bench_nanogpt.py): 4 layers, 4 heads, 128-wide, block 64,
batch 32, betas (0.9, 0.95), lr 3e-4, weight decay 0.1 on matrices,
gradient clipping at 1.0.  The text is synthetic (a seeded word-level Markov
chain rendered as characters); nothing is downloaded.
"""

import math

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

STEPS = 1000
EVAL_EVERY = 100
BLOCK, BATCH = 64, 32
N_LAYER, N_HEAD, N_EMBD = 4, 4, 128
LR, BETAS, WD, CLIP = 3e-4, (0.9, 0.95), 0.1, 1.0


def synthetic_text(n_chars=400_000, seed=0):
    """A word-level Markov chain over 300 pseudo-words, rendered as characters."""
    rng = np.random.default_rng(seed)
    letters = np.array(list("abcdefghijklmnopqrstuvwxyz"))
    words = ["".join(rng.choice(letters, size=rng.integers(2, 8))) for _ in range(300)]
    # each word has 5 likely successors (Zipf-like), plus a small uniform floor
    trans = np.full((300, 300), 0.02 / 300)
    for i in range(300):
        succ = rng.choice(300, size=5, replace=False)
        trans[i, succ] += 0.98 * np.array([0.4, 0.25, 0.15, 0.12, 0.08])
    trans /= trans.sum(axis=1, keepdims=True)
    out, w, total = [], 0, 0
    while total < n_chars:
        s = words[w] + (". " if rng.random() < 0.1 else " ")
        out.append(s)
        total += len(s)
        w = rng.choice(300, p=trans[w])
    text = "".join(out)[:n_chars]
    chars = sorted(set(text))
    data = torch.tensor([chars.index(c) for c in text], dtype=torch.long)
    return data, len(chars)


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.ln1 = nn.LayerNorm(N_EMBD)
        self.qkv = nn.Linear(N_EMBD, 3 * N_EMBD)
        self.proj = nn.Linear(N_EMBD, N_EMBD)
        self.ln2 = nn.LayerNorm(N_EMBD)
        self.fc = nn.Linear(N_EMBD, 4 * N_EMBD)
        self.out = nn.Linear(4 * N_EMBD, N_EMBD)

    def forward(self, x):
        b, t, c = x.shape
        q, k, v = self.qkv(self.ln1(x)).split(N_EMBD, dim=2)
        q, k, v = (z.view(b, t, N_HEAD, c // N_HEAD).transpose(1, 2) for z in (q, k, v))
        att = (q @ k.transpose(-2, -1).contiguous()) / math.sqrt(c // N_HEAD)
        mask = torch.ones(t, t, device=x.device, dtype=torch.bool).tril()
        att = att.masked_fill(~mask, float("-inf")).softmax(dim=-1)
        y = (att @ v).transpose(1, 2).reshape(b, t, c)
        x = x + self.proj(y)
        return x + self.out(F.gelu(self.fc(self.ln2(x))))


class TinyGPT(nn.Module):
    def __init__(self, vocab):
        super().__init__()
        self.wte = nn.Embedding(vocab, N_EMBD)
        self.wpe = nn.Embedding(BLOCK, N_EMBD)
        self.blocks = nn.ModuleList(Block() for _ in range(N_LAYER))
        self.ln_f = nn.LayerNorm(N_EMBD)
        self.head = nn.Linear(N_EMBD, vocab, bias=False)
        self.head.weight = self.wte.weight          # tied, as in nanoGPT
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, 0.0, 0.02)
            if isinstance(m, nn.Linear) and m.bias is not None:
                nn.init.zeros_(m.bias)

    def forward(self, idx, targets):
        x = self.wte(idx) + self.wpe(torch.arange(idx.shape[1], device=idx.device))
        for blk in self.blocks:
            x = blk(x)
        logits = self.head(self.ln_f(x))
        return F.cross_entropy(logits.view(-1, logits.shape[-1]), targets.view(-1))


def groups(params, lr=LR):
    """Two param groups as in nanoGPT: weight decay on matrices only."""
    decay = [p for p in params if p.dim() >= 2]
    no_decay = [p for p in params if p.dim() < 2]
    return [dict(params=decay, lr=lr, betas=BETAS, eps=1e-8, weight_decay=WD),
            dict(params=no_decay, lr=lr, betas=BETAS, eps=1e-8, weight_decay=0.0)]


def batches(data, seed, device="cpu"):
    """Endless random (x, y) windows of `data`, from a seeded generator."""
    g = torch.Generator().manual_seed(seed)
    while True:
        ix = torch.randint(len(data) - BLOCK - 1, (BATCH,), generator=g)
        x = torch.stack([data[i:i + BLOCK] for i in ix])
        y = torch.stack([data[i + 1:i + BLOCK + 1] for i in ix])
        yield x.to(device), y.to(device)


def setup(device="cpu"):
    """The model's seeded start: (model, train data, held-out batches)."""
    torch.manual_seed(1234)
    data, vocab = synthetic_text()
    split = int(0.9 * len(data))
    train, val = data[:split], data[split:]
    gen = batches(val, 99, device)
    val_batches = [next(gen) for _ in range(4)]
    return TinyGPT(vocab).to(device), train, val_batches


@torch.no_grad()
def evaluate(model, val_batches):
    return sum(float(model(x, y)) for x, y in val_batches) / len(val_batches)
