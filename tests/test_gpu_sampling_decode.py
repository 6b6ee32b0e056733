"""GPU: sampled decoding (AR sampling, speculative rejection sampling in both self-spec variants) on the
tiny hybrid.

- The batched sampled draft-then-verify step is checked teacher-forced against the oracle: every draw,
  every unmasking choice, every q row and the acceptance of each step follow oracle/accept.py on the
  logits and uniforms the GPU step used (decisions within 1e-6 of flipping are skipped).
- Sampled self-spec reproduces the AR sampling distribution (the pattern of the reference test
  inference/zoro-1/mlx/tests/test_tiny.py:253-286).
"""
import random
from collections import Counter

import numpy as np
import pytest
import torch

from oracle import accept as A
from trida_stack_amd.decode import DecodeStats, SamplingParams, ar_generate, selfspec_generate
from trida_stack_amd.model import HybridConfig, build_runtime
from trida_stack_amd.sampling import SampledBlockSpecStep, Sampler, prefill_batch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CFG = HybridConfig.tiny()


def prompt(n, seed=1):
    rng = random.Random(seed)
    return [rng.randrange(0, CFG.vocab - 10) for _ in range(n)]


def collect(gen):
    out = []
    for chunk in gen:
        out += chunk
    return out


def check_step_trace(trace, block, per, T, k, p, mask):
    """Replays one SampledBlockSpecStep on the oracle from the tensors the GPU step used: the draws of
    the still-masked slots, the choice of the slots to unmask, their q rows and the acceptance."""
    passes, ver = trace[:-1], trace[-1]
    B, _, V = passes[0]["lf"].shape
    q_ref = np.zeros((B, block, V))
    skipped = 0
    for pi, tr in enumerate(passes):
        lf, u, x = tr["lf"].cpu().numpy(), tr["u"].cpu().numpy(), tr["x"].cpu().numpy()
        midx, slots = tr["midx"].cpu().numpy(), tr["slots"].cpu().numpy()
        n = lf.shape[1]
        P, info = A.truncated_probs(lf, T, k, p, mask, return_info=True)
        for b in range(B):
            assert (np.diff(midx[b]) > 0).all()  # the masked slots, ascending
            for i in range(n):
                tok, gap = A.sample_inverse_cdf(P[b, i], float(u[b * n + i]))
                if gap > 1e-6 and info.boundary_gap[b, i] > 1e-6:
                    assert x[b, i] == tok, (pi, b, i)
                else:
                    skipped += 1
            conf = np.array([P[b, i, x[b, i]] for i in range(n)])
            order = sorted(range(n), key=lambda i: (-conf[i], midx[b, i]))
            chosen = [int(midx[b, i]) for i in order[: per[pi]]]
            border = [conf[i] for i in order[per[pi] - 1: per[pi] + 1]]
            if len(border) < 2 or abs(border[0] - border[1]) > 1e-6:
                assert sorted(slots[b].tolist()) == sorted(chosen), (pi, b)
            for i in range(n):
                if midx[b, i] in slots[b]:
                    q_ref[b, midx[b, i]] = P[b, i]
    q = ver["q"].cpu().numpy()
    assert np.abs(q - q_ref).max() < 2e-6
    res = A.rejection_accept(ver["pf"].cpu().numpy(), q, ver["drafts"].cpu().numpy(), ver["ua"].cpu().numpy(),
                             ver["us"].cpu().numpy(), temperature=T, top_k=k, top_p=p, mask_id=mask)
    return res, skipped


@pytest.mark.parametrize("T,k,p", [(0.7, 0, 0.95), (1.0, 20, 0.9)])
def test_sampled_blockspec_step_vs_oracle(gpu, T, k, p):
    rt = build_runtime(CFG, seed=3, device="cuda:0", embed_scale=8.0)
    B, block, denoise = 3, 8, 3
    prompts = [prompt(n, seed=10 + n) for n in (9, 17, 30)]
    cache = rt.make_cache(B, max_len=128)
    smp = Sampler(SamplingParams(temperature=T, top_k=k, top_p=p, seed=5), rt.dev, ban_id=rt.mask_id)
    logits = prefill_batch(rt, cache, prompts)
    step = SampledBlockSpecStep(rt, cache, block, denoise, smp)
    step.t0.copy_(smp.draw(logits))
    for _ in range(4):
        step.trace = []
        length_before = cache.length.clone()
        step.run()
        res, _ = check_step_trace(step.trace, block, step.per, T, k, p, rt.mask_id)
        n_acc, tok = step.n_acc.cpu().numpy(), step.token.cpu().numpy()
        ok = ~res["tie"]
        assert (n_acc[ok] == res["n_acc"][ok]).all() and (tok[ok] == res["token"][ok]).all()
        # ragged rollback: each sequence keeps the pending token and its accepted drafts
        assert torch.equal(cache.length.cpu(), (length_before + 1 + step.n_acc).cpu())
        assert (tok != rt.mask_id).all()
    smp.check()


def test_sample_rows_vs_oracle(gpu):
    """Draws from given truncation statistics: the inverse CDF at each row's uniform (near-ties skipped)."""
    from trida_stack_amd import kernels as TK

    rng = np.random.default_rng(3)
    for T, k, p in [(0.7, 0, 0.95), (1.0, 20, 0.9), (1.3, 0, 1.0)]:
        lf = (rng.normal(size=(3, 7, 5000)) * 3).astype(np.float32)
        u = rng.random(21).astype(np.float32)
        x = torch.from_numpy(lf).to(DEV)
        st = TK.truncate_stats(x, temperature=T, top_k=k, top_p=p, ban_id=11)
        tok = TK.sample_rows(x, st, torch.from_numpy(u).to(DEV), temperature=T, ban_id=11).cpu().numpy()
        P, info = A.truncated_probs(lf, T, k, p, 11, return_info=True)
        for r in range(21):
            b, i = divmod(r, 7)
            ref, gap = A.sample_inverse_cdf(P[b, i], float(u[r]))
            if gap > 1e-6 and info.boundary_gap[b, i] > 1e-6:
                assert tok[b, i] == ref, (T, k, p, r)
            assert tok[b, i] != 11 and P[b, i, tok[b, i]] > 0


def test_sampled_generate_runs(gpu):
    rt = build_runtime(CFG, seed=1, device="cuda:0", embed_scale=4.0)
    sp = SamplingParams(temperature=0.8, top_k=20, top_p=0.9, seed=3)
    for kw in ({}, {"denoise_steps": 2}):
        n = 4 if not kw else 8
        st = DecodeStats()
        out = collect(selfspec_generate(rt, rt.make_cache(1, max_len=256), prompt(12), max_new_tokens=30,
                                        eos_ids=set(), sp=sp, mask_id=rt.mask_id, n=n, stats=st, **kw))
        assert len(out) == 30 and rt.mask_id not in out
        assert st.forwards > 0
    out = collect(ar_generate(rt, rt.make_cache(1, max_len=256), prompt(12), max_new_tokens=20, eos_ids=set(),
                              sp=sp))
    assert len(out) == 20 and rt.mask_id not in out


def test_sampled_selfspec_preserves_distribution(gpu):
    """Sampled self-spec must reproduce the AR sampling distribution of the 4th generated token. Random
    models rarely accept drafts, so the MASK rows are patched to reuse the neighbouring row's logits
    (any q is valid for speculative sampling, and this one is often accepted)."""
    rt = build_runtime(CFG, seed=2, device="cuda:0", embed_scale=4.0)
    pr = prompt(10, seed=2)
    mask = rt.mask_id
    orig = rt.canvas

    def patched(cache, toks, n_clean, rows=None, as_float=True):
        L = orig(cache, toks, n_clean, rows=rows, as_float=as_float)
        idx = [i if (i == 0 or toks[i] != mask) else i - 1 for i in range(L.shape[0])]
        return L[torch.as_tensor(idx, device=L.device)]

    def hist(fn, reps, seed0, **kw):
        c, acc = Counter(), [0] * 4
        for i in range(reps):
            sp = SamplingParams(temperature=1.0, top_k=4, top_p=0.9, seed=seed0 + i)
            st = DecodeStats()
            out = collect(fn(rt, rt.make_cache(1, max_len=64), pr, max_new_tokens=4, eos_ids=set(), sp=sp, stats=st,
                             **kw))
            c[out[3]] += 1
            if st.accept_hist:
                acc = [a + b for a, b in zip(acc, st.accept_hist)]
        return c, acc

    R = 500
    a, _ = hist(ar_generate, R, 5000)
    a2, _ = hist(ar_generate, R, 90000)
    rt.canvas = patched
    b, acc = hist(selfspec_generate, R, 7000, mask_id=mask, n=4)
    tv = lambda x, y: 0.5 * sum(abs(x[t] - y[t]) for t in set(x) | set(y)) / R
    assert sum(acc[1:]) > R // 4, acc  # the accept path really ran
    assert tv(a, b) < max(0.08, 2.0 * tv(a, a2)), (tv(a, b), tv(a, a2))
