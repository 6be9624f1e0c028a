"""Synthetic Llama-style decoder for end-to-end determinism checks.

A torch restatement of the reference's benchmark model (reference
bench/bench.py:108-162: RMSNorm, q/k/v/o projections, causal GQA attention,
SiLU-gated MLP, residual adds, final norm and vocabulary head) and of its
determinism check (bench/bench.py:217-246): the logits of one sequence must
have the same bits whether it runs alone or inside a larger batch.

Under ``batch_invariant_mode`` every projection runs the invariant GEMM and
attention runs the invariant kernel; RMSNorm, SiLU, the embedding and the
residual adds are stock torch, which computes them per row with a fixed
reduction (tests/test_gpu_stock_ops.py guards that). Weights are random:
there is no checkpoint. They are drawn on the device from torch's seeded
generator, so the same seed gives the same model.
"""

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class DecoderConfig:
    hidden: int = 4096
    inter: int = 11008
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    layers: int = 32
    vocab: int = 32000
    eps: float = 1e-5


# random-init Llama-style decoder, 32 layers, hidden 4096,
# 32/8 heads, FFN 11008, vocabulary 32000.
LLAMA_7B_SHAPE = DecoderConfig()


class Block(torch.nn.Module):
    def __init__(self, c, device, dtype):
        super().__init__()
        kw = dict(bias=False, device=device, dtype=dtype)
        self.c = c
        self.q = torch.nn.Linear(c.hidden, c.heads * c.head_dim, **kw)
        self.k = torch.nn.Linear(c.hidden, c.kv_heads * c.head_dim, **kw)
        self.v = torch.nn.Linear(c.hidden, c.kv_heads * c.head_dim, **kw)
        self.o = torch.nn.Linear(c.heads * c.head_dim, c.hidden, **kw)
        self.gate = torch.nn.Linear(c.hidden, c.inter, **kw)
        self.up = torch.nn.Linear(c.hidden, c.inter, **kw)
        self.down = torch.nn.Linear(c.inter, c.hidden, **kw)
        self.n1 = torch.nn.RMSNorm(c.hidden, eps=c.eps, device=device, dtype=dtype)
        self.n2 = torch.nn.RMSNorm(c.hidden, eps=c.eps, device=device, dtype=dtype)

    def forward(self, x):
        c = self.c
        B, L, _ = x.shape
        y = self.n1(x)
        q = self.q(y).view(B, L, c.heads, c.head_dim).transpose(1, 2)
        k = self.k(y).view(B, L, c.kv_heads, c.head_dim).transpose(1, 2)
        v = self.v(y).view(B, L, c.kv_heads, c.head_dim).transpose(1, 2)
        a = F.scaled_dot_product_attention(q, k, v, is_causal=L > 1,
                                           scale=1.0 / math.sqrt(c.head_dim), enable_gqa=True)
        x = x + self.o(a.transpose(1, 2).reshape(B, L, c.heads * c.head_dim))
        y = self.n2(x)
        return x + self.down(F.silu(self.gate(y)) * self.up(y))


class Decoder(torch.nn.Module):
    def __init__(self, c, device, dtype):
        super().__init__()
        self.c = c
        self.embed = torch.nn.Embedding(c.vocab, c.hidden, device=device, dtype=dtype)
        self.blocks = torch.nn.ModuleList(Block(c, device, dtype) for _ in range(c.layers))
        self.norm = torch.nn.RMSNorm(c.hidden, eps=c.eps, device=device, dtype=dtype)
        self.head = torch.nn.Linear(c.hidden, c.vocab, bias=False, device=device, dtype=dtype)

    def forward(self, ids):
        """Logits of the last position of every sequence, (B, vocab)."""
        x = self.embed(ids)
        for blk in self.blocks:
            x = blk(x)
        return self.head(self.norm(x[:, -1]))


def build(config=LLAMA_7B_SHAPE, device="cuda", dtype=torch.bfloat16, seed=0):
    """Random-init decoder: nn.Linear / nn.Embedding default initialisation
    drawn on `device` after torch.manual_seed(seed)."""
    torch.manual_seed(seed)
    with torch.no_grad():
        m = Decoder(config, torch.device(device), dtype)
    return m.eval().requires_grad_(False)


def prompts(config, batch, length, seed=0, device="cuda"):
    """Token ids (batch, length): row 0 is the probe sequence, the other rows
    are unrelated sequences, all from a CPU generator seeded `seed`."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, config.vocab, (batch, length), generator=g).to(device)


def logits_bits(model, ids, invariant):
    """Bit pattern of row 0's last-position logits, with or without
    batch_invariant_mode."""
    from . import batch_invariant_mode

    with torch.no_grad():
        if invariant:
            with batch_invariant_mode():
                y = model(ids)
        else:
            y = model(ids)
    return y[0].contiguous().view(torch.int16 if y.dtype != torch.float32 else torch.int32)


def determinism(model, length=512, batches=(2, 4, 8), seed=0, invariant=True):
    """{batch: number of logits of sequence 0 whose bits differ from batch 1}."""
    c = model.c
    device = next(model.parameters()).device
    ids = prompts(c, max(batches), length, seed=seed, device=device)
    base = logits_bits(model, ids[:1], invariant)
    return {B: int((logits_bits(model, ids[:B], invariant) != base).sum()) for B in batches}
