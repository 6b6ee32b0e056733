"""Writes the GDN golden fixtures (tests/golden/*.npz) from transformers' torch implementations.

The reference declares transformers' Qwen3.5 torch functions as its CPU path for the linear-attention
layers (train/models/hybrid.py:31-35) and ships no fixtures for them, so these vectors are produced
here from the installed third-party package (transformers 5.15.0 in this image; the reference pins
4.57.6 in requirements-lock.txt:264 — the functions used, torch_chunk_gated_delta_rule,
torch_recurrent_gated_delta_rule, causal_conv1d_update and l2norm, are the same algorithm in both).
Inputs are fp32 holding bf16-representable values; outputs are fp32.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

from transformers.models.qwen3_5 import modeling_qwen3_5 as M

OUT = Path(__file__).resolve().parent


def bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def gdr_case(seed: int, B: int, T: int, H: int, Dk: int, Dv: int):
    g0 = torch.Generator().manual_seed(seed)
    q = bf(torch.randn(B, T, H, Dk, generator=g0))
    k = bf(torch.randn(B, T, H, Dk, generator=g0))
    v = bf(torch.randn(B, T, H, Dv, generator=g0))
    g = -F.softplus(torch.randn(B, T, H, generator=g0))
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g0))
    s0 = torch.randn(B, H, Dk, Dv, generator=g0) * 0.1  # transformers layout [B, H, Dk, Dv]
    return q, k, v, g, beta, s0


def main():
    torch.set_num_threads(4)
    # recurrent form, l2norm inside (use_qk_l2norm_in_kernel=True), 2 sequences, 19 rows
    q, k, v, g, beta, s0 = gdr_case(1, 2, 19, 3, 32, 16)
    o, sT = M.torch_recurrent_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state=s0.clone(),
                                               output_final_state=True, use_qk_l2norm_in_kernel=True)
    np.savez_compressed(OUT / "gdr_recurrent_tf.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(), g=g.numpy(),
                        beta=beta.numpy(), s0=s0.numpy(), o=o.float().numpy(), sT=sT.float().numpy())
    # chunked form, 150 rows (two full chunks of 64 and a padded tail), chunk 64
    q, k, v, g, beta, s0 = gdr_case(2, 1, 150, 2, 32, 32)
    o, sT = M.torch_chunk_gated_delta_rule(q, k, v, g=g, beta=beta, chunk_size=64, initial_state=s0.clone(),
                                           output_final_state=True, use_qk_l2norm_in_kernel=True)
    np.savez_compressed(OUT / "gdr_chunk_tf.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(), g=g.numpy(),
                        beta=beta.numpy(), s0=s0.numpy(), o=o.float().numpy(), sT=sT.float().numpy())
    # depthwise causal conv + SiLU with a conv state (the cached-decode form), 5 rows, 24 channels
    g0 = torch.Generator().manual_seed(3)
    C, K, T = 24, 4, 5
    x = bf(torch.randn(1, C, T, generator=g0))
    state = bf(torch.randn(1, C, K - 1, generator=g0))
    w = bf(torch.randn(C, K, generator=g0) * 0.5)
    st = state.clone()
    y = M.causal_conv1d_update(x, st, w, None, "silu")
    np.savez_compressed(OUT / "conv_tf.npz", x=x.numpy(), state=state.numpy(), w=w.numpy(),
                        y=y.float().numpy(), new_state=st.numpy())
    # l2norm
    xl = bf(torch.randn(4, 7, 32, generator=g0) * 3)
    np.savez_compressed(OUT / "l2norm_tf.npz", x=xl.numpy(), y=M.l2norm(xl, dim=-1, eps=1e-6).numpy())
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main()
