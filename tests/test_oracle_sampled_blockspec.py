"""CPU: the oracle's sampled draft-then-verify step (oracle.model.blockspec_sample_step) reproduces the
causal sampling distribution. Speculative rejection sampling is exact only when every draft follows
the q row kept for it given the drafts before it; the step unmasks slots in ascending order, fixed
before anything is drawn (the property the reference's canvas algorithm has, decode.py:361-378).

The test is exact on the causal side: the distributions of the first generated tokens are summed over
every truncated-distribution prefix (top-k 3). The step side is sampled many times over one cached
prefix; forwards are memoised on (committed tokens, block, mode), so thousands of steps cost a few
hundred forwards. A planted draw-dependent slot choice (keep the slots whose draws are most probable)
must fail the same check, so the test can tell the two apart.
"""
import copy

import numpy as np
import pytest
import torch

from oracle import accept as A
from oracle import model as OM
from trida_stack_amd.model import HybridConfig, init_weights

T, TOP_K, TOP_P = 3.0, 3, 1.0
PROMPT = [17, 43, 99, 5, 250, 61, 7, 180, 33, 12]


class MemoHybrid(OM.CpuHybrid):
    """CpuHybrid whose non-persisting forwards are memoised (results depend only on the committed
    tokens and the block). `draft_as_verify` runs draft passes token-causally instead, which makes the
    drafts close to the verify distribution (long accepted runs; any q is valid for the test)."""

    def __init__(self, cfg, w, draft_as_verify=False):
        super().__init__(cfg, w)
        self.memo = {}
        self.draft_as_verify = draft_as_verify

    def forward(self, tokens, cache, mode, n_clean=0):
        if mode == "causal":
            return super().forward(tokens, cache, mode, n_clean)
        if mode == "draft" and self.draft_as_verify:
            mode = "verify"
        key = (tuple(cache.tokens), tuple(tokens), mode, n_clean)
        hit = self.memo.get(key)
        if hit is None:
            logits = super().forward(tokens, cache, mode, n_clean)
            hit = self.memo[key] = (logits, cache.pending)
        cache.pending = hit[1]
        return hit[0].clone()


def biased_step(m, cache, t0, block, denoise, rng):
    """The planted mistake: every pass draws all still-masked slots and keeps the per-pass quota whose
    draws are most probable (a slot choice that depends on the draws, and later slots fixed first)."""
    mask = m.mask_id
    canvas, masked = [t0] + [mask] * block, [True] * block
    per = [block // denoise + (1 if p < block % denoise else 0) for p in range(denoise)]
    q = np.zeros((block, m.cfg.vocab))
    for p in range(denoise):
        L = m.forward(canvas, cache, "draft")
        cache.pending = None
        live = [j for j in range(block) if masked[j]]
        P = A.truncated_probs(L[live].numpy(), T, TOP_K, TOP_P, mask)
        u = rng.random(len(live))
        x = [A.sample_inverse_cdf(P[i], float(u[i]))[0] for i in range(len(live))]
        order = sorted(range(len(live)), key=lambda i: (-P[i, x[i]], live[i]))
        for i in order[: per[p]]:
            canvas[1 + live[i]], masked[live[i]] = x[i], False
            q[live[i]] = P[i]
    L = m.forward(canvas, cache, "verify")
    res = A.rejection_accept(L[None].numpy(), q[None], np.asarray([canvas[1:]], np.int64), rng.random((1, block)),
                             rng.random(1), temperature=T, top_k=TOP_K, top_p=TOP_P, mask_id=mask)
    acc, tok = int(res["n_acc"][0]), int(res["token"][0])
    m.commit(cache, 1 + acc)
    return canvas[1: 1 + acc] + [tok], tok, acc


def model(draft_as_verify):
    cfg = HybridConfig.tiny()
    return MemoHybrid(cfg, init_weights(cfg, seed=2, embed_scale=4.0), draft_as_verify)


def exact_causal(m, base, logits0, n):
    """Exact distributions [n, V] of generated tokens 0..n-1 under truncated causal sampling after the
    prompt held by `base` (logits0: its last-token logits)."""
    V = m.cfg.vocab
    out = np.zeros((n, V))

    def walk(prefix, logits, w, depth):
        P = A.truncated_probs(logits[None].numpy(), T, TOP_K, TOP_P, m.mask_id)[0]
        out[depth] += w * P
        if depth + 1 == n:
            return
        for x in np.nonzero(P)[0]:
            L = m.forward(prefix + [int(x)], base, "verify")
            base.pending = None
            walk(prefix + [int(x)], L[-1], w * P[x], depth + 1)

    walk([], logits0, 1.0, 0)
    return out


def sampled(m, base, logits0, step, n, reps, block, denoise, seed):
    """Histograms [n, V] of generated tokens 0..n-1: the first from the prompt logits, then steps."""
    V = m.cfg.vocab
    hist = np.zeros((n, V))
    rng = np.random.default_rng(seed)
    P0 = A.truncated_probs(logits0[None].numpy(), T, TOP_K, TOP_P, m.mask_id)[0]
    for _ in range(reps):
        cache = copy.deepcopy(base)
        t0 = A.sample_inverse_cdf(P0, float(rng.random()))[0]
        out = [t0]
        while len(out) < n:
            emit, t0, _ = step(m, cache, t0, block, denoise, rng)
            out += emit
        for i in range(n):
            hist[i, out[i]] += 1
    return hist / reps


def tv(p, q):
    return 0.5 * np.abs(p - q).sum(-1)


def oracle_step(m, cache, t0, block, denoise, rng):
    return OM.blockspec_sample_step(m, cache, t0, block, denoise, temperature=T, top_k=TOP_K, top_p=TOP_P, rng=rng)


@pytest.fixture(scope="module")
def setups():
    out = {}
    for dav in (False, True):
        m = model(dav)
        base = m.make_cache()
        out[dav] = (m, base, m.prefill(base, PROMPT))
    return out


REPS = 2000


@pytest.mark.parametrize("draft_as_verify,block,denoise", [(False, 2, 1), (False, 3, 2), (True, 3, 3)])
def test_sampled_step_preserves_causal_distribution(setups, draft_as_verify, block, denoise):
    m, base, logits0 = setups[draft_as_verify]
    n = 3
    ref = exact_causal(m, base, logits0, n)
    got = sampled(m, base, logits0, oracle_step, n, REPS, block, denoise, seed=block * 10 + denoise)
    d = tv(ref, got)
    # sampling noise of an empirical distribution over <= 27 outcomes from 2000 draws: TV ~ 0.02-0.03
    assert (d < 0.06).all(), d


def test_draw_dependent_slot_choice_is_detected(setups):
    """The planted mistake shifts the distribution of the first drafted token well beyond the noise."""
    m, base, logits0 = setups[True]
    n = 3
    ref = exact_causal(m, base, logits0, n)
    got = sampled(m, base, logits0, biased_step, n, REPS, 3, 3, seed=1)
    d = tv(ref, got)
    assert d.max() > 0.1, d
