"""CPU oracle: gated-delta-net (GDN) layer pieces. Test infrastructure only.

Recurrent state layout: [B, Hv, Dv, Dk] fp32 (row v holds S[:, v] over k), the layout of the MLX
runtime's GDNState.ssm (inference/zoro-1/mlx/trida_mlx/model.py:146-147). transformers keeps the
transpose [B, H, Dk, Dv]; `to_tf_state` / `from_tf_state` convert.

Restated from:
  gates           beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias)            [tf]:497-502
  l2norm          x * rsqrt(sum(x^2) + 1e-6)                                            [tf]:242-245
  causal conv     depthwise width-K conv over [window ++ x] + SiLU; window = last K-1 rows [tf]:200-239
  recurrence      S = e^g S; kv = S k; S += k ((v - kv) beta)^T; o = S^T (scale q)       [tf]:331-383
  chunked (WY)    chunk-parallel form of the same recurrence, chunk 64                  [tf]:249-328
  canvas readout  rows < num_clean token-causal, later rows read the block-end state,
                  s_clean = state after the clean rows  (causal_mode 2)  inference/zoro-1/mlx/trida_mlx/kernels.py:19-97
  restore/commit  state after the first `a` block rows from the block-entry snapshot;
                  conv window = last K-1 rows of (snapshot window ++ pre-conv rows[:a])  model.py:486-507
  block-bidir     per block, mean of the causal readout and a reversed within-block scan from the
                  block-entry state; state carried on causally          train/models/hybrid.py:461-536
([tf] = transformers/models/qwen3_5/modeling_qwen3_5.py, the reference's declared CPU fallback for
these layers, train/models/hybrid.py:31-35.)
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def to_tf_state(s: torch.Tensor) -> torch.Tensor:
    return s.transpose(-1, -2).contiguous()


from_tf_state = to_tf_state


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    x = x.float()
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def gates(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """(g, beta) fp32 [..., Hv] from the in_proj_a / in_proj_b outputs."""
    beta = torch.sigmoid(b.float())
    g = -torch.exp(A_log.float()) * F.softplus(a.float() + dt_bias.float())
    return g, beta


def causal_conv(x: torch.Tensor, window: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
    """x [B, T, C] pre-conv rows, window [B, K-1, C], weight [C, K], bias [C] or None (the conv1d bias
    of the layer, qwen3_5_diffusion.py:2211-2212).
    Returns (silu(conv) rounded to bf16 [B, T, C] fp32, new window [B, K-1, C] = last K-1 rows)."""
    K = weight.shape[1]
    full = torch.cat([window.float(), x.float()], dim=1)  # [B, K-1+T, C]
    T = x.shape[1]
    y = torch.zeros(x.shape[0], T, x.shape[2])
    if bias is not None:
        y += bias.float()
    w = weight.float()
    for j in range(K):
        y += full[:, j: j + T, :] * w[:, j]
    y = bf16_round(F.silu(y))
    return y, full[:, -(K - 1):, :].clone()


def prep(mixed_qkv, window, conv_w, a, b, A_log, dt_bias, Hk: int, Hv: int, Dk: int, Dv: int, conv_bias=None):
    """Conv + SiLU + split + l2norm(q, k) + gates for one GDN layer input block.
    Returns q, k [B,T,Hk,Dk] (unit-norm, bf16-rounded), v [B,T,Hv,Dv] (bf16-rounded), g, beta [B,T,Hv]
    fp32 and the new conv window."""
    B, T, _ = mixed_qkv.shape
    y, new_window = causal_conv(mixed_qkv, window, conv_w, conv_bias)
    q, k, v = torch.split(y, [Hk * Dk, Hk * Dk, Hv * Dv], dim=-1)
    q = bf16_round(l2norm(q.reshape(B, T, Hk, Dk)))
    k = bf16_round(l2norm(k.reshape(B, T, Hk, Dk)))
    v = v.reshape(B, T, Hv, Dv)
    g, beta = gates(a, b, A_log, dt_bias)
    return q, k, v, g, beta, new_window


def _expand_heads(x: torch.Tensor, Hv: int) -> torch.Tensor:
    """GQA: value head h reads key head h // (Hv / Hk) (repeat_interleave, [tf]:503-505)."""
    Hk = x.shape[2]
    return x if Hk == Hv else x.repeat_interleave(Hv // Hk, dim=2)


def recurrent(q, k, v, g, beta, state: Optional[torch.Tensor] = None, scale: Optional[float] = None,
              record_states: bool = False):
    """Token-by-token gated delta rule. q,k [B,T,Hk,Dk], v [B,T,Hv,Dv], g,beta [B,T,Hv] (g = log decay),
    state [B,Hv,Dv,Dk]. Returns (o [B,T,Hv,Dv] fp32, final state, list of states after each row)."""
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2], v.shape[3]
    scale = Dk ** -0.5 if scale is None else scale
    q = _expand_heads(q.float(), Hv) * scale
    k = _expand_heads(k.float(), Hv)
    v, g, beta = v.float(), g.float(), beta.float()
    S = torch.zeros(B, Hv, Dv, Dk) if state is None else state.float().clone()
    out = torch.zeros(B, T, Hv, Dv)
    states = []
    for t in range(T):
        S = S * torch.exp(g[:, t])[:, :, None, None]
        kv = (S * k[:, t, :, None, :]).sum(-1)                      # [B,Hv,Dv]
        delta = (v[:, t] - kv) * beta[:, t, :, None]
        S = S + delta[:, :, :, None] * k[:, t, :, None, :]
        out[:, t] = (S * q[:, t, :, None, :]).sum(-1)
        if record_states:
            states.append(S.clone())
    return out, S, states


def chunked(q, k, v, g, beta, state: Optional[torch.Tensor] = None, scale: Optional[float] = None,
            chunk: int = 64):
    """Chunk-parallel (WY / UT) form of `recurrent`. Within a chunk with cumulative log decay G:
        A0[i,j] = -beta_i (k_i . k_j) e^{G_i - G_j}  (j < i),  T = (I - A0)^{-1}
        W = T (beta k e^{G}),  U = T (beta v)
        v_new = U - W S,  o = (q e^{G}) S + [(q k^T) e^{G_i - G_j}]_{j<=i} v_new
        S' = e^{G_last} S + (k e^{G_last - G})^T v_new
    Returns (o [B,T,Hv,Dv] fp32, final state)."""
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2], v.shape[3]
    scale = Dk ** -0.5 if scale is None else scale
    q = _expand_heads(q.float(), Hv).transpose(1, 2) * scale         # [B,H,T,Dk]
    k = _expand_heads(k.float(), Hv).transpose(1, 2)
    v = v.float().transpose(1, 2)
    g = g.float().transpose(1, 2)                                    # [B,H,T]
    beta = beta.float().transpose(1, 2)
    S = torch.zeros(B, Hv, Dv, Dk) if state is None else state.float().clone()
    out = torch.zeros(B, Hv, T, Dv)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        qc, kc, vc = q[:, :, c0:c1], k[:, :, c0:c1], v[:, :, c0:c1]
        G = torch.cumsum(g[:, :, c0:c1], dim=-1)                     # [B,H,C]
        bc = beta[:, :, c0:c1]
        C = c1 - c0
        diff = G[..., :, None] - G[..., None, :]
        lower = torch.tril(torch.ones(C, C, dtype=torch.bool), diagonal=-1)
        incl = torch.tril(torch.ones(C, C, dtype=torch.bool))
        decay = torch.where(incl, torch.exp(torch.where(incl, diff, torch.zeros_like(diff))), torch.zeros_like(diff))
        A0 = torch.where(lower, -(bc[..., :, None] * (kc @ kc.transpose(-1, -2)) * decay), torch.zeros_like(diff))
        eye = torch.eye(C).expand_as(A0)
        Tm = torch.linalg.solve_triangular(eye - A0, eye, upper=False, unitriangular=True)
        W = Tm @ (bc[..., None] * kc * torch.exp(G)[..., None])      # [B,H,C,Dk]
        U = Tm @ (bc[..., None] * vc)                                # [B,H,C,Dv]
        St = S.transpose(-1, -2)                                     # [B,H,Dk,Dv]
        v_new = U - W @ St
        attn = (qc @ kc.transpose(-1, -2)) * decay
        out[:, :, c0:c1] = (qc * torch.exp(G)[..., None]) @ St + attn @ v_new
        glast = G[..., -1:]
        St = St * torch.exp(glast)[..., None] + (kc * torch.exp(glast - G)[..., None]).transpose(-1, -2) @ v_new
        S = St.transpose(-1, -2)
    return out.transpose(1, 2).contiguous(), S


def canvas(q, k, v, g, beta, state, num_clean: int, causal_mode: int = 2, scale: Optional[float] = None):
    """Block-causal canvas readout over T rows starting from `state` (never modified).
    causal_mode 1: every row token-causal. causal_mode 2: rows < num_clean token-causal, rows >=
    num_clean read the block-end state. Returns (o fp32 [B,T,Hv,Dv], s_clean = state after
    min(num_clean, T) rows, s_end = state after all T rows)."""
    T = k.shape[1]
    o, s_end, states = recurrent(q, k, v, g, beta, state, scale, record_states=True)
    nc = max(0, min(num_clean, T))
    s_clean = state.float().clone() if nc == 0 else states[nc - 1]
    if causal_mode == 2 and nc < T:
        Hv = v.shape[2]
        Dk = k.shape[3]
        sc = Dk ** -0.5 if scale is None else scale
        qm = _expand_heads(q[:, nc:].float(), Hv) * sc                # [B,T',Hv,Dk]
        o[:, nc:] = torch.einsum("bhvk,bthk->bthv", s_end, qm)
    return o, s_clean, s_end


def restore(snap_state, snap_window, k, v, g, beta, preconv, n_keep):
    """Rollback to an accepted prefix of the block: per sequence b, the state after the first
    n_keep[b] rows from the block-entry snapshot, and the conv window = last K-1 rows of
    (snapshot window ++ preconv[:n_keep]). q is not needed (no readout)."""
    B = k.shape[0]
    Km1 = snap_window.shape[1]
    keep = [int(n) for n in n_keep]
    states = snap_state.float().clone()
    for a in sorted(set(keep) - {0}):  # the sequences that keep a rows advance together
        idx = torch.tensor([b for b in range(B) if keep[b] == a])
        _, s, _ = recurrent(k[idx, :a], k[idx, :a], v[idx, :a], g[idx, :a], beta[idx, :a], snap_state[idx])
        states[idx] = s
    windows = [torch.cat([snap_window[b].float(), preconv[b, :keep[b]].float()], dim=0)[-Km1:] for b in range(B)]
    return states, torch.stack(windows)


def block_bidirectional(q, k, v, g, beta, state: Optional[torch.Tensor], block_size: int,
                        scale: Optional[float] = None):
    """Block-local-bidirectional readout (train/models/hybrid.py:461-536, _block_bidirectional_gdr), blocks
    of block_size consecutive rows (the last may be shorter). For a block with causal entry state E:
    out_f = the causal readout, out_b = the readout of a scan over the block's rows in reverse order
    starting from E, out = (out_f + out_b) / 2; the state carried to the next block (and returned) is
    the causal one. Returns (o fp32 [B,T,Hv,Dv], final state)."""
    T = k.shape[1]
    B, Hv, Dv, Dk = v.shape[0], v.shape[2], v.shape[3], k.shape[3]
    S = torch.zeros(B, Hv, Dv, Dk) if state is None else state.float().clone()
    out = torch.zeros(B, T, Hv, Dv)
    for t0 in range(0, T, block_size):
        t1 = min(T, t0 + block_size)
        o_f, S_next, _ = recurrent(q[:, t0:t1], k[:, t0:t1], v[:, t0:t1], g[:, t0:t1], beta[:, t0:t1], S, scale)
        rev = torch.arange(t1 - 1, t0 - 1, -1)
        o_b, _, _ = recurrent(q[:, rev], k[:, rev], v[:, rev], g[:, rev], beta[:, rev], S, scale)
        out[:, t0:t1] = 0.5 * (o_f + o_b.flip(1))
        S = S_next
    return out, S
