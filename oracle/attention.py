"""CPU oracle: canvas attention over a KV cache with the draft / verify / mixed masks. Test
infrastructure only.

Mask (inference/zoro-1/mlx/trida_mlx/model.py:461-470): the committed prefix is visible to every
canvas row; inside the block, row t sees block column j when
  verify / causal (mode 0)        j <= t
  draft / bidirectional (mode 1)  always                       (the noisy MASK rows see the whole block)
  canvas / mixed (mode 2)         j <= t for t < n_clean, else always   (`(c <= r) | (r >= n_clean)`)
Attention itself is the Qwen3.5 SDPA with GQA (query head h reads KV head h // (Hq/Hkv)) and the
output gate `out * sigmoid(gate)` ([tf]:629-701, model.py:263-280).
"""
from __future__ import annotations

from typing import Optional

import torch

MODES = {"verify": 0, "causal": 0, "draft": 1, "bidirectional": 1, "canvas": 2, "mixed": 2}


def canvas_mask(prefix_len: int, T: int, mode: int, n_clean: int = 0) -> torch.Tensor:
    """Boolean [T, prefix_len + T] visibility mask."""
    r = torch.arange(T)[:, None]
    c = torch.arange(T)[None, :]
    if mode == 0:
        inner = c <= r
    elif mode == 1:
        inner = torch.ones(T, T, dtype=torch.bool)
    else:
        inner = (c <= r) | (r >= n_clean)
    pre = torch.ones(T, prefix_len, dtype=torch.bool)
    return torch.cat([pre, inner], dim=1)


def canvas_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, prefix_len,
                     mode: int, n_clean: int = 0, scale: Optional[float] = None,
                     gate: Optional[torch.Tensor] = None) -> torch.Tensor:
    """q [B, T, Hq, D]; k_cache, v_cache [B, Hkv, Lmax, D] holding the block's keys at
    [prefix, prefix + T); prefix_len per sequence. Returns fp32 [B, T, Hq, D]; with gate
    ([B, T, Hq, D]) the output is bf16(attn) * sigmoid(gate)."""
    B, T, Hq, D = q.shape
    Hkv = k_cache.shape[1]
    G = Hq // Hkv
    scale = D ** -0.5 if scale is None else scale
    out = torch.zeros(B, T, Hq, D)
    for b in range(B):
        p = int(prefix_len[b])
        n = p + T
        k = k_cache[b, :, :n].float().repeat_interleave(G, dim=0)      # [Hq, n, D]
        v = v_cache[b, :, :n].float().repeat_interleave(G, dim=0)
        s = torch.einsum("thd,hnd->htn", q[b].float(), k) * scale       # [Hq, T, n]
        m = canvas_mask(p, T, mode, n_clean)
        s = s.masked_fill(~m[None], float("-inf"))
        pr = torch.softmax(s, dim=-1)
        out[b] = torch.einsum("htn,hnd->thd", pr, v)
    if gate is not None:
        out = out.to(torch.bfloat16).float() * torch.sigmoid(gate.float())
    return out
