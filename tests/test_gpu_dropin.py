"""GPU: the drop-in decode surface. Banned / gated tokens (apply_ban, decode.py:76-99) against the oracle's
restatement; greedy self-spec == greedy AR under a ban with the banned ids never emitted; the engine's
reference defaults (sampled decoding), prompt-cache reuse and progress callback."""
import random

import numpy as np
import pytest
import torch

from oracle import accept as A
from trida_stack_amd import kernels as K
from trida_stack_amd.decode import DecodeStats, LogitRules, SamplingParams, ar_generate, selfspec_generate
from trida_stack_amd.engine import Engine
from trida_stack_amd.model import HybridConfig, TridaRuntime, init_weights

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CFG = HybridConfig.tiny()


def prompt(n, seed=1):
    rng = random.Random(seed)
    return [rng.randrange(0, CFG.vocab - 10) for _ in range(n)]


def collect(gen):
    out = []
    for ch in gen:
        out.extend(ch)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ban_and_gate_match_oracle(gpu, dtype):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(3, 33, 5000, generator=g) * 3).to(dtype)
    # make some gated tokens likely so that both outcomes of the gate occur
    x[:, ::2, 17] += 12
    x[:, 1::3, 4000] += 9
    x[:, 1::2, 3] += 11  # a banned token holding much of the mass: the raw and the banned rows' softmax differ
    banned = (3, 4999, 17000, -2, 3)
    gate = ((17, 0.5), (4000, 0.2), (123, 0.0), (9999, 0.3))
    ref = A.apply_ban(x.float().numpy(), banned, gate)
    # the notes take the raw row's probabilities (_gate_note, decode.py:63-73, gets the unbanned logits);
    # the gate decides on the banned row (apply_ban, decode.py:88-98)
    ref_p = A.gate_probs(x.float().numpy(), gate)
    assert np.abs(ref_p - A.gate_probs(A.apply_ban(x.float().numpy(), banned), gate)).max() > 0.1
    xd = x.to(DEV)
    rules = LogitRules(SamplingParams(banned=banned, gate=gate, gate_log=[]), DEV)
    raw = rules.raw_buffer(3 * 33, DEV)
    rules.apply(xd, raw)
    got = xd.float().cpu().numpy()
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin], ref[fin])  # nothing else is touched
    gp = raw.cpu().numpy().reshape(3, 33, len(gate))
    assert np.abs(gp - ref_p).max() < 1e-5
    # the decisions were not all one way
    assert np.isneginf(ref[..., 17]).any() and np.isfinite(ref[..., 17]).any()


def test_ban_rows_of_a_strided_block(gpu):
    """Rows of a view ([B, T, V] slice of rows) are banned in place; other rows are untouched."""
    x = torch.zeros(2, 6, 100, device=DEV, dtype=torch.bfloat16)
    K.ban_tokens(x[1, 2:5], torch.tensor([0, 99], device=DEV))
    ninf = torch.isneginf(x.float()).cpu()
    assert ninf[1, 2:5][:, [0, 99]].all() and ninf.sum() == 6


@pytest.fixture(scope="module")
def rt():
    r = TridaRuntime(CFG, init_weights(CFG, seed=0, embed_scale=4.0), device=DEV)
    r.gdr_form = "recurrent"  # verify rows run the AR arithmetic: greedy self-spec == greedy AR bit for bit
    return r


def test_greedy_selfspec_equals_ar_under_ban(gpu, rt):
    g = SamplingParams(temperature=0.0)
    p = prompt(25, seed=3)
    free = collect(ar_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=40, eos_ids=set(), sp=g))
    common = [t for t, _ in sorted(((t, -free.count(t)) for t in set(free)), key=lambda z: z[1])][:2]
    sp = SamplingParams(temperature=0.0, banned=tuple(common) + (CFG.vocab + 5,))
    ar = collect(ar_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=40, eos_ids=set(), sp=sp))
    assert not set(common) & set(ar) and ar != free
    for n, d in ((4, 0), (8, 2)):
        ss = collect(selfspec_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=40, eos_ids=set(), sp=sp,
                                       mask_id=CFG.mask_id, n=n, denoise_steps=d))
        assert ss == ar, (n, d)


def test_sampled_decoding_never_emits_banned(gpu, rt):
    p = prompt(20, seed=4)
    g = SamplingParams(temperature=0.0)
    free = collect(ar_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=30, eos_ids=set(), sp=g))
    ban = tuple(sorted(set(free)))[:6]
    for n, d in ((None, None), (4, 0), (8, 2)):
        sp = SamplingParams(temperature=0.8, top_k=20, top_p=0.9, seed=3, banned=ban)
        if n is None:
            out = collect(ar_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=40, eos_ids=set(), sp=sp))
        else:
            out = collect(selfspec_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=40, eos_ids=set(),
                                            sp=sp, mask_id=CFG.mask_id, n=n, denoise_steps=d))
        assert len(out) == 40 and not set(ban) & set(out), (n, d)


def test_gate_blocks_and_logs(gpu, rt):
    """A gate above every probability the model gives a token blocks it everywhere, and the exact causal
    rows where the token had raw probability >= 0.05 are logged."""
    g = SamplingParams(temperature=0.0)
    p = prompt(25, seed=3)
    free = collect(ar_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=30, eos_ids=set(), sp=g))
    tok = max(set(free), key=free.count)
    log = []
    sp = SamplingParams(temperature=0.0, gate=((tok, 1.01),), gate_log=log)
    for n, d in ((4, 0), (8, 2)):
        log.clear()
        out = collect(selfspec_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=30, eos_ids=set(), sp=sp,
                                        mask_id=CFG.mask_id, n=n, denoise_steps=d))
        assert tok not in out, (n, d)
        assert log and all(0.05 <= q < 1.01 and thr == 1.01 for q, thr in log), (n, d)


def test_engine_defaults_cache_and_progress(gpu, rt):
    eng = Engine(rt, mode="self-spec", gen_block=4, prefill_chunk=16)
    p = prompt(40, seed=8)
    seen = []
    st = DecodeStats()
    out = collect(eng.generate_ids(p, max_tokens=20, stats=st, progress=lambda d, t: seen.append((d, t))))
    assert len(out) == 20 and st.mode.startswith("self-spec") and st.reused_tokens == 0
    assert seen and seen[-1] == (40, 40) and [d for d, _ in seen] == [16, 32, 40]  # prefill chunks of 16
    # default sampling is SamplingParams(): seeds left unset give different continuations
    out2 = collect(eng.generate_ids(p, max_tokens=20))
    assert len(out2) == 20
    # prompt cache: a follow-up prompt that extends what the live cache holds reuses it
    g = SamplingParams(temperature=0.0)
    base = collect(eng.generate_ids(p, max_tokens=12, sampling=g))
    held = list(eng.cache.tokens[0])
    follow = held + prompt(9, seed=9)
    st = DecodeStats()
    a = collect(eng.generate_ids(follow, max_tokens=16, sampling=g, stats=st))
    assert st.reused_tokens == len(held) and st.prompt_tokens == len(follow)
    fresh = Engine(rt, mode="self-spec", gen_block=4, prompt_cache=False)
    st2 = DecodeStats()
    b = collect(fresh.generate_ids(follow, max_tokens=16, sampling=g, stats=st2))
    assert st2.reused_tokens == 0
    # the same tokens (a resumed recurrent state and a fresh chunked prefill round differently, so a
    # first divergence is tolerated only where the causal top-2 gap is below 0.1)
    if a != b:
        i = next(i for i, (x, y) in enumerate(zip(a, b)) if x != y)
        c = rt.make_cache(max_len=512)
        top2 = torch.topk(rt.prefill(c, follow + b[:i]), 2).values
        assert float(top2[0] - top2[1]) < 0.1
    assert eng.cached_tokens()[0] > 0
