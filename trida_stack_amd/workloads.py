"""Seeded synthetic inputs at the benchmark shapes of the self-spec step.

Every generator draws on the CPU from ``torch.Generator().manual_seed(seed)`` so a GPU run and a CPU
check see identical values; callers move the tensors where they need them.
"""
from __future__ import annotations

import math

import torch


def geometric_prefix(g: torch.Generator, p: float, cap: int, n: int) -> torch.Tensor:
    """n draws of Geometric(p) on {0, 1, ...} (failures before the first success), capped at cap."""
    u = torch.rand(n, generator=g, dtype=torch.float64).clamp_min(1e-300)
    L = torch.floor(torch.log(u) / math.log1p(-p)).to(torch.int64)
    return L.clamp(max=cap)


def greedy_accept_inputs(seed: int = 0, batch: int = 1, block: int = 32, vocab: int = 151936,
                         ctx: int = 4096, p: float = 0.15):
    """Greedy acceptance on synthetic verify logits.

    logits [B, block + 1, V] fp32 ~ N(0, 4) (std 2); for each sequence the first L drafts equal the
    row argmax, L ~ Geometric(p) capped at block, draft L (if any) is a random non-argmax id and the
    rest are uniform random ids. ctx_len = ctx for every sequence.
    Returns dict(logits, drafts, ctx_len, prefix_len).
    """
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(batch, block + 1, vocab, generator=g) * 2.0
    am = logits.argmax(dim=-1)
    L = geometric_prefix(g, p, block, batch)
    drafts = torch.randint(0, vocab, (batch, block), generator=g)
    for b in range(batch):
        n = int(L[b])
        drafts[b, :n] = am[b, :n]
        if n < block:
            off = int(torch.randint(1, vocab, (1,), generator=g))
            drafts[b, n] = (am[b, n] + off) % vocab
    ctx_len = torch.full((batch,), ctx, dtype=torch.int64)
    return dict(logits=logits, drafts=drafts, ctx_len=ctx_len, prefix_len=L)
