"""The C1 reference case as test infrastructure: a 2-layer decoder-only
transformer (d_model 128, 4 heads, FFN 512 GELU, LayerNorm, vocab 1024,
seq 64), N(0, 0.02) init from a seed, fp32; next-token cross-entropy per
sequence.  Provides factor capture (inputs and output gradients of every
linear layer, biases included) and per-sample autograd gradients."""

from __future__ import annotations

import torch
from torch import nn

D_MODEL, HEADS, FFN, VOCAB, SEQ = 128, 4, 512, 1024, 64


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.ln1 = nn.LayerNorm(D_MODEL)
        self.q = nn.Linear(D_MODEL, D_MODEL)
        self.k = nn.Linear(D_MODEL, D_MODEL)
        self.v = nn.Linear(D_MODEL, D_MODEL)
        self.o = nn.Linear(D_MODEL, D_MODEL)
        self.ln2 = nn.LayerNorm(D_MODEL)
        self.fc1 = nn.Linear(D_MODEL, FFN)
        self.fc2 = nn.Linear(FFN, D_MODEL)

    def forward(self, x):
        b, t, _ = x.shape
        h = self.ln1(x)
        q = self.q(h).view(b, t, HEADS, -1).transpose(1, 2)
        k = self.k(h).view(b, t, HEADS, -1).transpose(1, 2)
        v = self.v(h).view(b, t, HEADS, -1).transpose(1, 2)
        att = (q @ k.transpose(-1, -2)) / (q.shape[-1] ** 0.5)
        mask = torch.ones(t, t, dtype=torch.bool).tril()
        att = att.masked_fill(~mask, float("-inf")).softmax(-1)
        y = (att @ v).transpose(1, 2).reshape(b, t, D_MODEL)
        x = x + self.o(y)
        return x + self.fc2(torch.nn.functional.gelu(self.fc1(self.ln2(x))))


class TinyDecoder(nn.Module):
    def __init__(self, seed: int = 0):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.tok = nn.Embedding(VOCAB, D_MODEL)
        self.pos = nn.Embedding(SEQ, D_MODEL)
        self.blocks = nn.ModuleList([Block(), Block()])
        self.ln_f = nn.LayerNorm(D_MODEL)
        self.head = nn.Linear(D_MODEL, VOCAB)
        with torch.no_grad():
            for p in self.parameters():
                if p.dim() >= 2 or p.shape[0] in (VOCAB, D_MODEL, FFN):
                    p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
            for m in self.modules():
                if isinstance(m, nn.LayerNorm):
                    m.weight.fill_(1.0)
                    m.bias.zero_()

    def forward(self, ids):
        x = self.tok(ids) + self.pos(torch.arange(ids.shape[1]))[None]
        for blk in self.blocks:
            x = blk(x)
        return self.head(self.ln_f(x))

    def linears(self):
        return [(n, m) for n, m in self.named_modules() if isinstance(m, nn.Linear)]


def per_sequence_loss(model, ids):
    """(B,) next-token cross-entropy, mean over each sequence's positions."""
    logits = model(ids)
    ce = torch.nn.functional.cross_entropy(
        logits[:, :-1].reshape(-1, VOCAB), ids[:, 1:].reshape(-1), reduction="none")
    return ce.view(ids.shape[0], -1).mean(1)


def capture_factors(model, ids):
    """{layer: (a (B,T,in), g (B,T,out))} for every linear, from one backward
    of the summed per-sequence losses (so sample i's rows carry dL_i/dy)."""
    acts, grads, hooks = {}, {}, []
    for name, m in model.linears():
        hooks.append(m.register_forward_hook(lambda _m, inp, _o, n=name: acts.__setitem__(n, inp[0].detach())))
        hooks.append(m.register_full_backward_hook(
            lambda _m, _gi, go, n=name: grads.__setitem__(n, go[0].detach())))
    model.zero_grad()
    per_sequence_loss(model, ids).sum().backward()
    for h in hooks:
        h.remove()
    return {n: (acts[n], grads[n]) for n, _ in model.linears()}


def per_sample_grads(model, ids):
    """(B, P) flattened [weight, bias] gradients of every linear, one backward per sample."""
    rows = []
    for i in range(ids.shape[0]):
        model.zero_grad()
        per_sequence_loss(model, ids[i : i + 1]).sum().backward()
        parts = []
        for _n, m in model.linears():
            parts.append(torch.cat([m.weight.grad, m.bias.grad[:, None]], dim=1).flatten())
        rows.append(torch.cat(parts))
    return torch.stack(rows)


def c1_inputs(seed: int = 0):
    """(model, train ids (32, 64), query ids (8, 64)), token ids uniform over the vocab."""
    model = TinyDecoder(seed)
    gen = torch.Generator().manual_seed(seed + 1)
    train = torch.randint(0, VOCAB, (32, SEQ), generator=gen)
    query = torch.randint(0, VOCAB, (8, SEQ), generator=gen)
    return model, train, query
