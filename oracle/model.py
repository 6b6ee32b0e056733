"""CPU oracle: the hybrid decoder and the self-spec decode loops. Test infrastructure only (and the
bench's timed CPU baseline).

Follows the reference runtime inference/zoro-1/mlx/trida_mlx/model.py (forwards, canvas, commit) and
decode.py (ar_generate, selfspec_generate), one sequence at a time, in fp32 arithmetic with bf16
rounding where the model stores bf16 (GEMM outputs, residual stream, normalised activations). The
layer math is the Qwen3.5 decoder layer ([tf]:420-760): zero-centred RMSNorm, GDN layer (oracle.gdn),
full attention with per-head q/k RMSNorm, rotate-half partial RoPE, GQA and a sigmoid output gate,
SwiGLU MLP, tied LM head.

Also restates the vLLM plugin's greedy block-diffusion loop (qwen3_5_diffusion.py:449-632, 1180-1270):
shift_conf_pred, denoise_round, diffusion_generate.

Weights use the dict layout of trida_stack_amd.model.init_weights ([out, in] projections; the GDN
in-projection stacks [qkv | z | b | a] rows, the attention one [Hq x (q | gate) | k | v]).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch
import torch.nn.functional as F

from . import attention as OA
from . import gdn as OG


def bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, zero_centred: bool = True) -> torch.Tensor:
    y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    return bf(y * ((1.0 + w) if zero_centred else w))


def rope(x: torch.Tensor, pos: torch.Tensor, rot: int, theta: float) -> torch.Tensor:
    """Rotate-half RoPE on the first `rot` dims. x [T, H, D], pos [T]."""
    half = rot // 2
    i = torch.arange(half, dtype=torch.float32)
    inv = theta ** (-2.0 * i / rot)
    ang = pos.float()[:, None] * inv[None, :]                      # [T, half]
    cs, sn = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:rot]
    out = x.clone()
    out[..., :half] = x1 * cs - x2 * sn
    out[..., half:rot] = x2 * cs + x1 * sn
    return out


@dataclass
class CpuCache:
    kv: Dict[int, tuple] = field(default_factory=dict)       # attention layer -> (K [Hkv, L, D], V)
    state: Dict[int, torch.Tensor] = field(default_factory=dict)   # GDN layer -> [1, Hv, Dv, Dk]
    window: Dict[int, torch.Tensor] = field(default_factory=dict)  # GDN layer -> [1, Kc-1, C]
    tokens: List[int] = field(default_factory=list)
    pending: Optional[dict] = None

    @property
    def length(self) -> int:
        return len(self.tokens)


class CpuHybrid:
    # causal (persisting) GDN layers run the chunked WY form (oracle.gdn.chunked, pinned equal to the
    # token recurrence) instead of the token loop: the same states, faster over hundreds of rows
    gdn_chunked_causal = False

    def __init__(self, cfg, weights: Dict[str, torch.Tensor]):
        self.cfg = cfg
        self.w = {k: v.detach().to("cpu", torch.float32) for k, v in weights.items()}
        self.mask_id = cfg.mask_id

    def make_cache(self) -> CpuCache:
        c = self.cfg
        cache = CpuCache()
        for i in range(c.n_layers):
            if c.is_attention(i):
                cache.kv[i] = (torch.zeros(c.n_kv_heads, 0, c.head_dim), torch.zeros(c.n_kv_heads, 0, c.head_dim))
            else:
                cache.state[i] = torch.zeros(1, c.lin_v_heads, c.lin_v_dim, c.lin_k_dim)
                cache.window[i] = torch.zeros(1, c.conv_kernel - 1, c.conv_dim)
        return cache

    # ------------------------------------------------------------------ layers
    def _attention(self, i, x, cache: CpuCache, mode: int, n_clean: int, persist: bool):
        c, w = self.cfg, self.w
        p = f"l{i}."
        T = x.shape[0]
        D, Hq, Hkv = c.head_dim, c.n_heads, c.n_kv_heads
        qkv = bf(x @ w[p + "w_qkv"].t())
        qg = qkv[:, : 2 * Hq * D].reshape(T, Hq, 2 * D)
        q, gate = qg[..., :D], qg[..., D:]
        k = qkv[:, 2 * Hq * D: 2 * Hq * D + Hkv * D].reshape(T, Hkv, D)
        v = qkv[:, 2 * Hq * D + Hkv * D:].reshape(T, Hkv, D)
        pos = torch.arange(cache.length, cache.length + T)
        q = bf(rope(rmsnorm(q, w[p + "q_norm"], c.rms_eps), pos, c.rot_dim, c.rope_theta))
        k = bf(rope(rmsnorm(k, w[p + "k_norm"], c.rms_eps), pos, c.rot_dim, c.rope_theta))
        K0, V0 = cache.kv[i]
        Kc = torch.cat([K0, k.transpose(0, 1)], dim=1)
        Vc = torch.cat([V0, v.transpose(0, 1)], dim=1)
        if persist:
            cache.kv[i] = (Kc, Vc)
        o = OA.canvas_attention(q[None], Kc[None], Vc[None], [cache.length], mode, n_clean, gate=gate[None])[0]
        return bf(bf(o).reshape(T, -1) @ w[p + "w_o"].t()), (k, v)

    def _gdn(self, i, x, cache: CpuCache, gdn_mode: int, n_clean: int, persist: bool):
        proj = self.gdn_proj(i, x)
        y, rec = self.gdn_core(i, proj, cache, gdn_mode, n_clean, persist)
        return self.gdn_out(i, y, proj), rec

    def gdn_proj(self, i, x):
        """The GDN layer's in-projection of the normed rows x [T, hidden]: [T, C + VD + 2 Hv] rows stacking
        the pre-conv q|k|v, z, b and a (bf16-valued)."""
        return bf(x @ self.w[f"l{i}.w_in"].t())

    def gdn_core(self, i, proj, cache: CpuCache, gdn_mode: int, n_clean: int, persist: bool):
        """Conv + gates + the gated delta rule of GDN layer i on its projection rows: the readout y
        [T, Hv, Dv] (bf16-valued) and, unless persisted, the rows a commit needs."""
        c, w = self.cfg, self.w
        p = f"l{i}."
        C, VD, Hv = c.conv_dim, c.value_dim, c.lin_v_heads
        xpre = proj[None, :, :C]
        b_in = proj[None, :, C + VD: C + VD + Hv]
        a_in = proj[None, :, C + VD + Hv: C + VD + 2 * Hv]
        q, k, v, g, beta, new_win = OG.prep(xpre, cache.window[i], w[p + "conv_w"], a_in, b_in, w[p + "A_log"],
                                            w[p + "dt_bias"], c.lin_k_heads, Hv, c.lin_k_dim, c.lin_v_dim)
        if persist:
            if self.gdn_chunked_causal:
                o, s_end = OG.chunked(q, k, v, g, beta, cache.state[i])
            else:
                o, s_end, _ = OG.recurrent(q, k, v, g, beta, cache.state[i])
            cache.state[i] = s_end
            cache.window[i] = new_win
            rec = None
        else:
            o, _, _ = OG.canvas(q, k, v, g, beta, cache.state[i], n_clean, causal_mode=gdn_mode)
            rec = (k, v, g, beta, xpre)
        return bf(o)[0], rec

    def gdn_out(self, i, y, proj):
        """Gated RMSNorm of the readout y [T, Hv, Dv] by z (from the projection rows) and the
        out-projection: the layer's residual branch [T, hidden]."""
        c, w = self.cfg, self.w
        p = f"l{i}."
        T = y.shape[0]
        z = proj[:, c.conv_dim: c.conv_dim + c.value_dim]
        yn = bf(y * torch.rsqrt((y * y).mean(-1, keepdim=True) + c.rms_eps))
        yn = bf(yn * w[p + "gnorm"] * F.silu(z.reshape(T, c.lin_v_heads, c.lin_v_dim)))
        return bf(yn.reshape(T, -1) @ w[p + "w_out"].t())

    _MODES = {"causal": (0, 1), "verify": (0, 1), "canvas": (2, 2), "draft": (1, 2)}

    def layer(self, i: int, h: torch.Tensor, cache: CpuCache, mode: str, n_clean: int):
        """Decoder layer i ([tf]:420-760) on the hidden rows h [T, hidden] of a block on top of `cache`:
        h + mixer(rmsnorm(h)), then + mlp(rmsnorm(.)). The mixer's mask / readout follow `mode` as in
        forward (n_clean: the canvas's clean rows; draft passes use 1). A causal layer persists its KV /
        GDN state into the cache; the others return the rows a commit needs. Returns (h', rec)."""
        c, w = self.cfg, self.w
        p = f"l{i}."
        att_mode, gdn_mode = self._MODES[mode]
        persist = mode == "causal"
        x = rmsnorm(h, w[p + "in_norm"], c.rms_eps)
        if c.is_attention(i):
            r, rec = self._attention(i, x, cache, att_mode, n_clean, persist)
        else:
            r, rec = self._gdn(i, x, cache, gdn_mode, n_clean, persist)
        return self.mlp(i, bf(h + r)), rec

    def mlp(self, i: int, h: torch.Tensor) -> torch.Tensor:
        """The second half of layer i: h + SwiGLU MLP(rmsnorm(h))."""
        return bf(h + self.mlp_branch(i, h))

    def mlp_branch(self, i: int, h: torch.Tensor) -> torch.Tensor:
        """SwiGLU MLP(rmsnorm(h)) of layer i: the branch added to h (bf16-valued)."""
        c, w = self.cfg, self.w
        p = f"l{i}."
        x = rmsnorm(h, w[p + "post_norm"], c.rms_eps)
        gu = bf(x @ w[p + "w_gu"].t())
        I = c.intermediate
        act = bf(F.silu(gu[:, :I]) * gu[:, I:])
        return bf(act @ w[p + "w_down"].t())

    def head(self, h: torch.Tensor) -> torch.Tensor:
        """Final RMSNorm and the (tied) LM head: bf16-valued fp32 logits [T, V]."""
        x = rmsnorm(h, self.w["final_norm"], self.cfg.rms_eps)
        return bf(x @ self.w.get("lm_head", self.w["embed"]).t())

    def forward(self, tokens: List[int], cache: CpuCache, mode: str, n_clean: int = 0) -> torch.Tensor:
        """mode: causal (persist), verify, canvas (n_clean) or draft. Returns bf16-valued fp32 logits [T, V]."""
        persist = mode == "causal"
        T = len(tokens)
        nc = {"causal": T, "verify": T, "canvas": n_clean, "draft": 1}[mode]
        h = self.w["embed"][torch.as_tensor(tokens)]
        recs = {}
        for i in range(self.cfg.n_layers):
            h, recs[i] = self.layer(i, h, cache, mode, nc)
        logits = self.head(h)
        if persist:
            cache.tokens.extend(tokens)
        else:
            cache.pending = {"recs": recs, "tokens": list(tokens)}
        return logits

    # ------------------------------------------------------------------ reference runtime API
    def prefill(self, cache: CpuCache, tokens: List[int]) -> torch.Tensor:
        return self.forward(tokens, cache, "causal")[-1]

    def ar_step(self, cache: CpuCache, tok: int) -> torch.Tensor:
        return self.forward([tok], cache, "causal")[-1]

    def canvas(self, cache: CpuCache, tokens: List[int], n_clean: int) -> torch.Tensor:
        return self.forward(tokens, cache, "canvas", n_clean)

    def commit(self, cache: CpuCache, adv: int) -> None:
        """Keep the first adv rows of the pending block (model.py:486-507)."""
        rec = cache.pending
        assert rec is not None and 1 <= adv <= len(rec["tokens"])
        c = self.cfg
        for i, r in rec["recs"].items():
            if c.is_attention(i):
                k, v = r
                K0, V0 = cache.kv[i]
                cache.kv[i] = (torch.cat([K0, k[:adv].transpose(0, 1)], 1), torch.cat([V0, v[:adv].transpose(0, 1)], 1))
            else:
                k, v, g, beta, xpre = r
                st, win = OG.restore(cache.state[i], cache.window[i], k, v, g, beta, xpre, [adv])
                cache.state[i], cache.window[i] = st, win
        cache.tokens.extend(rec["tokens"][:adv])
        cache.pending = None


# ---------------------------------------------------------------------- decode loops (greedy)
def argmax(x: torch.Tensor) -> int:
    return int(torch.argmax(x))


def ar_generate(m: CpuHybrid, prompt: List[int], max_new: int) -> List[int]:
    """Greedy AR decode (decode.py:273-293)."""
    cache = m.make_cache()
    logits = m.prefill(cache, prompt)
    out = []
    while True:
        tok = argmax(logits)
        out.append(tok)
        if len(out) >= max_new:
            return out
        logits = m.ar_step(cache, tok)


def selfspec_generate(m: CpuHybrid, prompt: List[int], max_new: int, n: int = 4):
    """Greedy self-spec with the bd_bidir_shift canvas (decode.py:297-387): cold start [t0, MASK x 2n-2],
    verify round [pending, specs, MASK x n-1] with n_clean = n. Returns (tokens, forwards)."""
    cache = m.make_cache()
    logits = m.prefill(cache, prompt)
    blk, K = 2 * n - 1, n - 1
    t0 = argmax(logits)
    out, fwd = [], 0
    t0_emitted = False
    pending = specs = None
    while len(out) < max_new:
        if specs is not None:
            L = m.canvas(cache, [pending] + specs + [m.mask_id] * (n - 1), n)
            fwd += 1
            vals = L.argmax(-1).tolist()
            acc = 0
            while acc < K and vals[acc] == specs[acc]:
                acc += 1
            if acc < K:
                m.commit(cache, 1 + acc)
                out += specs[:acc] + [vals[acc]]
                t0, t0_emitted, pending, specs = vals[acc], True, None, None
            else:
                m.commit(cache, n)
                out += specs + [vals[n - 1]]
                pending, specs = vals[n - 1], vals[n:blk]
        else:
            L = m.canvas(cache, [t0] + [m.mask_id] * (blk - 1), n)
            fwd += 1
            vals = L[:n].argmax(-1).tolist()
            m.commit(cache, 1)
            out += ([] if t0_emitted else [t0]) + [vals[0]]
            t0_emitted = True
            pending, specs = vals[0], vals[1:n]
    return out[:max_new], fwd


def blockspec_step(m: CpuHybrid, cache: CpuCache, t0: int, block: int, denoise: int):
    """One draft-then-verify step: `denoise` block-diffusion passes over [t0, MASK x block] (each unmasks
    the block/denoise most confident MASK slots, shift readout), a token-causal verify pass over
    [t0, d_1..d_block], greedy acceptance and rollback. Returns (emitted tokens, next t0, n_acc)."""
    canvas = [t0] + [m.mask_id] * block
    masked = [True] * block
    per = [block // denoise + (1 if p < block % denoise else 0) for p in range(denoise)]
    for p in range(denoise):
        L = m.forward(canvas, cache, "draft")
        cache.pending = None
        probs = torch.softmax(L[:block], dim=-1)
        conf, am = probs.max(dim=-1)
        cand = [(float(conf[j]), j) for j in range(block) if masked[j]]
        cand.sort(key=lambda x: (-x[0], x[1]))
        for _, j in cand[: per[p]]:
            canvas[1 + j] = int(am[j])
            masked[j] = False
    L = m.forward(canvas, cache, "verify")
    vals = L.argmax(-1).tolist()
    acc = 0
    while acc < block and vals[acc] == canvas[1 + acc]:
        acc += 1
    m.commit(cache, 1 + acc)
    return canvas[1: 1 + acc] + [vals[acc]], vals[acc], acc


def blockspec_generate(m: CpuHybrid, prompt: List[int], max_new: int, block: int = 32, denoise: int = 4):
    """Greedy draft-then-verify decode. The first token comes from the prompt logits; each step emits
    the accepted drafts plus the bonus token. Returns (tokens, steps)."""
    cache = m.make_cache()
    t0 = argmax(m.prefill(cache, prompt))
    out, steps = [t0], 0
    while len(out) < max_new:
        emit, t0, _ = blockspec_step(m, cache, t0, block, denoise)
        out += emit
        steps += 1
    return out[:max_new], steps


# ---------------------------------------------------------------------- sampled draft-then-verify
def blockspec_sample_step(m: CpuHybrid, cache: CpuCache, t0: int, block: int, denoise: int, *, temperature: float,
                          top_k: int, top_p: float, rng):
    """One sampled draft-then-verify step (the rejection-sampling counterpart of blockspec_step):
    `denoise` passes over [t0, MASK x block] that unmask the block in ascending slot order. Pass p
    takes the per[p] lowest still-masked slots; each slot j is drawn by inverse CDF from the truncated
    distribution P_j (decode.py:102-130; MASK banned, qwen3_5_diffusion.py:820) of its row of that pass's
    logits (row j predicts slot j), and P_j is kept as the slot's q row (the draft distribution,
    qwen3_5_diffusion.py:779). The slots a pass takes are fixed before the draws and each q depends only
    on lower slots, so every draft follows its q given the drafts before it, which is what makes the
    rejection sampling of the verify pass (oracle.accept.rejection_accept, decode.py:333-354) reproduce
    the causal distribution; the reference's canvas algorithm has the same property (its specs come
    from rows that see only lower positions, decode.py:361-378). Then a token-causal verify pass, the
    acceptance, and the rollback to 1 + n_acc rows. Uniforms come from the numpy Generator rng, in the
    order: per pass, one per drawn slot; then block acceptance uniforms and one correction/bonus uniform.
    Returns (emitted tokens, next t0, n_acc)."""
    import numpy as np

    from . import accept as A

    mask = m.mask_id
    canvas = [t0] + [mask] * block
    per = [block // denoise + (1 if p < block % denoise else 0) for p in range(denoise)]
    V = m.cfg.vocab
    q = np.zeros((block, V))
    s0 = 0
    for p in range(denoise):
        L = m.forward(canvas, cache, "draft")
        cache.pending = None
        slots = list(range(s0, s0 + per[p]))
        P = A.truncated_probs(L[slots].numpy(), temperature, top_k, top_p, mask)
        u = rng.random(len(slots))
        for i, j in enumerate(slots):
            canvas[1 + j] = A.sample_inverse_cdf(P[i], float(u[i]))[0]
            q[j] = P[i]
        s0 += per[p]
    L = m.forward(canvas, cache, "verify")
    res = A.rejection_accept(L[None].numpy(), q[None], np.asarray([canvas[1:]], np.int64), rng.random((1, block)),
                             rng.random(1), temperature=temperature, top_k=top_k, top_p=top_p, mask_id=mask)
    acc, tok = int(res["n_acc"][0]), int(res["token"][0])
    m.commit(cache, 1 + acc)
    return canvas[1: 1 + acc] + [tok], tok, acc


# ---------------------------------------------------------------------- pure block diffusion (greedy)
def shift_conf_pred(logits: torch.Tensor, mask_id: int):
    """Shifted readout of a canvas forward (qwen3_5_diffusion.py:449-466): position i >= 1 is
    predicted by the logits of position i-1, with its fp32 softmax maximum as the confidence; position
    0 (the seed) gets -inf / mask_id. logits [CL, V]. Returns (conf [CL] fp32, pred [CL] int64)."""
    probs = torch.softmax(logits[:-1].float(), dim=-1)
    c, p = probs.max(dim=-1)
    conf = torch.cat([torch.tensor([float("-inf")]), c])
    pred = torch.cat([torch.tensor([mask_id]), p])
    return conf, pred


def denoise_round(canvas: List[int], logits: torch.Tensor, mask_id: int, threshold: float) -> List[int]:
    """One LowConfidenceShift round (qwen3_5_diffusion.py:476-524, 596-600): every still-masked position
    (never position 0) whose confidence exceeds `threshold` takes its prediction; when masks remain but
    none passes, only the most confident masked position (first on ties) does."""
    conf, pred = shift_conf_pred(logits, mask_id)
    masked = [i >= 1 and t == mask_id for i, t in enumerate(canvas)]
    score = [float(conf[i]) if masked[i] else float("-inf") for i in range(len(canvas))]
    take = [s > threshold for s in score]
    if any(masked) and not any(take):
        best = max(range(len(canvas)), key=lambda i: (score[i], -i))
        take[best] = True
    return [int(pred[i]) if take[i] else t for i, t in enumerate(canvas)]


def diffusion_generate(m: CpuHybrid, prompt: List[int], max_new: int, canvas: int = 32, threshold: float = 0.9,
                       max_steps: Optional[int] = None) -> List[int]:
    """Greedy block diffusion (qwen3_5_diffusion.py:1180-1270): each block [seed, MASK x (canvas-1)] is
    denoised with draft passes (prefix + whole block visible, MASK rows read the block-end GDN state)
    until no mask is left or max_steps rounds ran; a causal forward then commits the block, every
    position of it is emitted, and the argmax of its last logit seeds the next block. The first seed
    is the argmax of the prompt's last logit."""
    max_steps = canvas if max_steps is None else max_steps
    cache = m.make_cache()
    seed = argmax(m.prefill(cache, prompt))
    out: List[int] = []
    while True:
        blk = [seed] + [m.mask_id] * (canvas - 1)
        for _ in range(max_steps):
            blk = denoise_round(blk, m.forward(blk, cache, "draft"), m.mask_id, threshold)
            cache.pending = None
            if m.mask_id not in blk[1:]:
                break
        logits = m.forward(blk, cache, "causal")
        out.extend(blk)
        if len(out) >= max_new:
            return out[:max_new]
        seed = argmax(logits[-1])
