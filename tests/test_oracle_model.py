"""Pins the CPU oracle of the hybrid decoder and the decode loops (the reference's own invariants,
inference/zoro-1/mlx/tests/test_tiny.py): canvas clean rows == AR logits, commit == AR state, greedy
self-spec == greedy AR."""
import random

import pytest
import torch

from oracle import model as OM
from trida_stack_amd.model import HybridConfig, init_weights

CFG = HybridConfig.tiny()


@pytest.fixture(scope="module")
def m():
    torch.manual_seed(0)
    return OM.CpuHybrid(CFG, init_weights(CFG, seed=0, embed_scale=4.0))


def prompt(n, seed=1):
    rng = random.Random(seed)
    return [rng.randrange(0, CFG.vocab - 10) for _ in range(n)]


def test_chunked_prefill_equals_one_shot(m):
    p = prompt(23)
    c1 = m.make_cache()
    l1 = m.prefill(c1, p)
    c2 = m.make_cache()
    m.prefill(c2, p[:9])
    l2 = m.prefill(c2, p[9:])
    assert torch.allclose(l1, l2, atol=0.05)


def test_canvas_clean_rows_are_ar_logits(m):
    n = 4
    p = prompt(15)
    cont = prompt(n, seed=7)
    c = m.make_cache()
    ar = [m.prefill(c, p)] + [m.ar_step(c, t) for t in cont]
    c2 = m.make_cache()
    m.prefill(c2, p)
    L = m.canvas(c2, cont + [CFG.mask_id] * (n - 1), n)
    for i in range(n):
        assert torch.allclose(L[i], ar[i + 1], atol=0.05), i


@pytest.mark.parametrize("adv", [1, 2, 4])
def test_commit_matches_ar_state(m, adv):
    n = 4
    p = prompt(12)
    cont = prompt(n, seed=3)
    c = m.make_cache()
    m.prefill(c, p)
    m.canvas(c, cont + [CFG.mask_id] * (n - 1), n)
    m.commit(c, adv)
    got = m.ar_step(c, 42)
    c2 = m.make_cache()
    m.prefill(c2, p + cont[:adv])
    ref = m.ar_step(c2, 42)
    assert torch.allclose(got, ref, atol=0.05)
    assert c.tokens == p + cont[:adv] + [42]


def test_greedy_selfspec_is_lossless(m):
    p = prompt(20, seed=11)
    ar = OM.ar_generate(m, p, 40)
    ss, fwd = OM.selfspec_generate(m, p, 40, n=4)
    assert ss == ar
    assert fwd <= len(ar)


def test_greedy_blockspec_is_lossless(m):
    p = prompt(20, seed=12)
    ar = OM.ar_generate(m, p, 30)
    bs, steps = OM.blockspec_generate(m, p, 30, block=8, denoise=2)
    assert bs == ar
