"""CPU oracle: self-spec acceptance (greedy and rejection sampling). Test infrastructure only.

Greedy follows TridaDiffusionSampler._selfspec_step's greedy branch
(inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:906-914) and the greedy verify of
selfspec_generate (inference/zoro-1/mlx/trida_mlx/decode.py:323-332).

Sampling follows truncated_probs (decode.py:102-130) and the sampled verify (decode.py:333-354):
accept draft i iff ratio >= 1 or u_i < ratio with ratio = p_i(d_i) / q_i(d_i) (0 where q = 0); the
accepted length is the first rejection; the correction is drawn from norm(max(0, P_i - q_i)) (P_i
when that mass is 0) and, when every draft is accepted, the bonus from P_K. The reference draws those
tokens with an RNG (mx.random.categorical) that has no uniform -> token contract, so this build
defines it: inverse CDF in vocabulary order with one uniform, token = min{x : cdf(x) > u}.
The vLLM path additionally bans the MASK id from every verify row (qwen3_5_diffusion.py:820);
``mask_id`` reproduces that (-1 = no ban).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np


# ------------------------------------------------------------------------------------------ greedy
def argmax_first(x: np.ndarray) -> np.ndarray:
    """argmax over the last axis with torch.argmax semantics: the first index wins ties and a NaN
    ranks above every number (the first NaN wins)."""
    x = np.asarray(x, dtype=np.float32)
    nan = np.isnan(x)
    filled = np.where(nan, np.float32(np.inf), x)
    am = np.argmax(filled, axis=-1)
    has_nan = nan.any(axis=-1)
    first_nan = np.argmax(nan, axis=-1)
    # a row with an +inf and a later NaN: the NaN wins
    return np.where(has_nan, first_nan, am).astype(np.int64)


def greedy_accept(logits: np.ndarray, drafts: np.ndarray, n_live: Optional[np.ndarray] = None,
                  ctx_len: Optional[np.ndarray] = None):
    """logits [B, R, V] fp32, drafts [B, K] int64 (R >= K + 1).

    Returns (am [B, R], n_acc [B], bonus [B], crop [B]) with
      am    = row argmax (shift readout: row j predicts canvas slot j + 1)
      match = (am[:, :K] == drafts) & (j < n_live)                     (qwen3_5_diffusion.py:908)
      n_acc = sum(cumprod(match))                                      (qwen3_5_diffusion.py:909-910)
      bonus = am[n_acc]                                                (qwen3_5_diffusion.py:912)
      crop  = ctx_len + 1 + n_acc  (KV kept: prefix, pending token, accepted drafts;
                                    decode.py:357 commits 1 + acc, model.py:490-492 trims the rest)
    """
    logits = np.asarray(logits, dtype=np.float32)
    drafts = np.asarray(drafts, dtype=np.int64)
    B, R, _ = logits.shape
    K = drafts.shape[1]
    assert R >= K + 1
    am = argmax_first(logits)
    live = np.full(B, K) if n_live is None else np.clip(np.asarray(n_live), 0, K)
    j = np.arange(K)
    match = (am[:, :K] == drafts) & (j[None, :] < live[:, None])
    n_acc = np.cumprod(match.astype(np.int64), axis=1).sum(axis=1) if K else np.zeros(B, np.int64)
    bonus = am[np.arange(B), n_acc]
    ctx = np.zeros(B, np.int64) if ctx_len is None else np.asarray(ctx_len, np.int64)
    return am, n_acc.astype(np.int32), bonus.astype(np.int64), ctx + 1 + n_acc


# ------------------------------------------------------------------------------------------ bans
def apply_ban(x: np.ndarray, banned=(), gate=()) -> np.ndarray:
    """apply_ban (inference/zoro-1/mlx/trida_mlx/decode.py:76-99) over the last axis: fp32 copy of x with
    every banned id at -inf, then for each gate (id, thr) with 0 <= id < V and thr > 0, x[..., id] = -inf
    where the id's probability under the softmax of the banned row, exp(x_id - logsumexp(x)), is below
    thr. The logsumexp is taken once, before the gates (decode.py:89); ``gate_probs`` gives those raw
    probabilities."""
    x = np.array(x, dtype=np.float32, copy=True)
    V = x.shape[-1]
    for i in banned:
        if 0 <= int(i) < V:
            x[..., int(i)] = -np.inf
    if gate:
        p_all = gate_probs(x, gate)
        for g, (tid, thr) in enumerate(gate):
            if 0 <= int(tid) < V and thr > 0:
                x[..., int(tid)] = np.where(p_all[..., g] < thr, np.float32(-np.inf), x[..., int(tid)])
    return x


def gate_probs(x: np.ndarray, gate) -> np.ndarray:
    """[..., n_gate] float64: exp(x[..., id] - logsumexp(x)) per gate (0 for an id outside [0, V) or a
    row with no finite value): the raw probability apply_ban compares with each gate's threshold."""
    x64 = np.asarray(x, np.float64)
    V = x64.shape[-1]
    m = np.max(x64, axis=-1, keepdims=True)
    finite = np.isfinite(m)
    mm = np.where(finite, m, 0.0)
    lse = (mm + np.log(np.sum(np.exp(x64 - mm), axis=-1, keepdims=True)))[..., 0]
    out = np.zeros(x64.shape[:-1] + (len(gate),))
    for g, (tid, _) in enumerate(gate):
        if 0 <= int(tid) < V:
            out[..., g] = np.where(finite[..., 0], np.exp(x64[..., int(tid)] - lse), 0.0)
    return out


# ------------------------------------------------------------------------------------------ sampling
@dataclass
class TruncInfo:
    """Per-row facts of a truncation, used by tests to recognise near-ties."""
    kept: np.ndarray        # [..., V] bool
    boundary_gap: np.ndarray  # [...] |cum_before(last kept) - top_p| style distance to the tie


def truncated_probs(logits: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0,
                    mask_id: int = -1, return_info: bool = False):
    """Top-k / top-p truncated sampling distribution over the last axis (decode.py:102-130).

    The logits are divided by the temperature in fp32 (as the reference does); the softmax, the
    nucleus cumulative mass and the renormalisation are done in float64 here, so this is the exact
    distribution up to the fp32 temperature division. Kept set: with top-k, every x >= the k-th
    largest value (ties kept, decode.py:114-116); the nucleus is then computed on exactly the k
    largest values (the sorted mx.topk list, decode.py:117-122), or on the whole sorted row without
    top-k (decode.py:123-128), keeping the sorted prefix whose mass *before* each value is < top_p
    (the value that crosses top_p stays); the final kept set is every x >= the last kept value, so
    ties at that value are all kept.
    """
    x = np.asarray(logits, dtype=np.float32).copy()
    if mask_id >= 0:
        x[..., mask_id] = -np.inf
    if temperature != 1.0:
        x = (x / np.float32(temperature)).astype(np.float32)
    V = x.shape[-1]
    x64 = x.astype(np.float64)
    flat = x64.reshape(-1, V)
    kept = np.isfinite(flat) | (flat == np.inf)
    gaps = np.full(flat.shape[0], np.inf)
    for r in range(flat.shape[0]):
        row = flat[r]
        order = np.argsort(-row, kind="stable")
        s = row[order]
        thr = -np.inf
        if 0 < top_k < V:
            thr = s[top_k - 1]
        if top_p < 1.0:
            cand = s[:top_k] if 0 < top_k < V else s
            m = cand[0]
            e = np.exp(cand - m)
            ps = e / e.sum()
            before = np.cumsum(ps) - ps
            keep = before < top_p
            n_keep = max(int(keep.sum()), 1)
            thr = max(thr, cand[n_keep - 1])
            gaps[r] = np.min(np.abs(before - top_p))
        kept[r] = row >= thr
    kept = kept.reshape(x.shape)
    m = np.max(np.where(kept, x64, -np.inf), axis=-1, keepdims=True)
    e = np.where(kept, np.exp(x64 - m), 0.0)
    P = e / e.sum(axis=-1, keepdims=True)
    if return_info:
        return P, TruncInfo(kept=kept, boundary_gap=gaps.reshape(x.shape[:-1]))
    return P


def sample_inverse_cdf(weights: np.ndarray, u: float) -> tuple[int, float]:
    """token = min{x : sum_{y<=x} w(y) > u * sum(w)} (vocabulary order). Returns (token, gap), gap
    being the distance of u*total to the nearest cdf step in the units of ``weights`` (probabilities
    here), for the tie tolerance of tests."""
    w = np.asarray(weights, dtype=np.float64)
    c = np.cumsum(w)
    tot = c[-1]
    t = u * tot
    tok = int(np.searchsorted(c, t, side="right"))
    tok = min(tok, len(w) - 1)
    # skip zero-weight tokens the search could land on at the very end
    while w[tok] <= 0 and tok > 0:
        tok -= 1
    gap = float(np.min(np.abs(c - t)))
    return tok, gap


def rejection_accept(p_logits: np.ndarray, q_probs: np.ndarray, drafts: np.ndarray,
                     u_accept: np.ndarray, u_sample: np.ndarray, *, temperature: float,
                     top_k: int = 0, top_p: float = 1.0, mask_id: int = -1,
                     ctx_len: Optional[np.ndarray] = None):
    """Sampled acceptance for a batch (decode.py:333-354).

    p_logits [B, R, V] verify logits (R >= K + 1), q_probs [B, K, V] the draft distributions the
    drafts [B, K] were drawn from, u_accept [B, K] and u_sample [B] uniforms in [0, 1).
    Returns dict(n_acc [B], token [B], crop [B], ratio [B, K], p_draft [B, K], q_draft [B, K],
    tie [B] bool: True where a decision is within 1e-6 of flipping (accept test, nucleus boundary
    or inverse-CDF step)).
    """
    p_logits = np.asarray(p_logits, np.float32)
    q = np.asarray(q_probs, np.float64)
    drafts = np.asarray(drafts, np.int64)
    B, R, V = p_logits.shape
    K = drafts.shape[1]
    assert R >= K + 1
    P, info = truncated_probs(p_logits[:, : K + 1], temperature, top_k, top_p, mask_id, return_info=True)
    n_acc = np.zeros(B, np.int64)
    token = np.zeros(B, np.int64)
    ratio = np.zeros((B, K))
    pd = np.zeros((B, K))
    qd = np.zeros((B, K))
    tie = np.zeros(B, bool)
    for b in range(B):
        for i in range(K):
            pd[b, i] = P[b, i, drafts[b, i]]
            qd[b, i] = q[b, i, drafts[b, i]]
            ratio[b, i] = pd[b, i] / max(qd[b, i], 1e-30) if qd[b, i] > 0 else 0.0
        acc = (ratio[b] >= 1.0) | (u_accept[b] < ratio[b])
        a = 0
        while a < K and acc[a]:
            a += 1
        n_acc[b] = a
        rows = range(0, min(a + 1, K))
        near = any(abs(u_accept[b, i] - ratio[b, i]) < 1e-6 or abs(ratio[b, i] - 1.0) < 1e-6 for i in rows)
        near |= bool(np.any(info.boundary_gap[b, : a + 1] < 1e-6))
        if a < K:
            r = np.maximum(P[b, a] - q[b, a], 0.0)
            if r.sum() <= 0:
                r = P[b, a]
        else:
            r = P[b, K]
        tok, gap = sample_inverse_cdf(r, float(u_sample[b]))
        token[b] = tok
        tie[b] = near or gap < 1e-6
    ctx = np.zeros(B, np.int64) if ctx_len is None else np.asarray(ctx_len, np.int64)
    return dict(n_acc=n_acc, token=token, crop=ctx + 1 + n_acc, ratio=ratio, p_draft=pd, q_draft=qd, tie=tie)
