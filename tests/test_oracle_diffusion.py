"""Oracle pins for the greedy block-diffusion loop (LowConfidenceShift commit gate,
inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:449-632, 1180-1270): the shifted
readout against an independent softmax, the commit gate on hand-made confidences, and the seed of every
block against a fresh causal prefill of everything emitted before it."""
import random

import numpy as np
import torch

from oracle import model as OM
from trida_stack_amd.model import HybridConfig, init_weights

MASK = 99


def logits_with_conf(rows):
    """[CL, V] logits whose softmax maxima are exactly the given (token, prob) per row, V = 8."""
    V = 8
    out = torch.full((len(rows), V), -1e4)
    for r, (tok, p) in enumerate(rows):
        # p on tok, the rest spread evenly: log-probabilities as logits
        rest = (1 - p) / (V - 1)
        out[r] = torch.log(torch.full((V,), rest))
        out[r, tok] = float(np.log(p))
    return out


def test_shift_readout_against_numpy_softmax():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, 50, generator=g) * 3
    conf, pred = OM.shift_conf_pred(x, MASK)
    assert conf[0] == float("-inf") and pred[0] == MASK
    xn = x.numpy().astype(np.float64)
    for i in range(1, 6):
        e = np.exp(xn[i - 1] - xn[i - 1].max())
        pr = e / e.sum()
        assert abs(float(conf[i]) - pr.max()) < 1e-6
        assert int(pred[i]) == int(np.argmax(pr))


def test_commit_gate():
    # positions: 0 seed, 1 committed, 2..4 masked
    canvas = [5, 6, MASK, MASK, MASK]
    # row r predicts position r+1: pos2 <- row1 (0.95), pos3 <- row2 (0.5), pos4 <- row3 (0.92)
    L = logits_with_conf([(1, 0.3), (2, 0.95), (3, 0.5), (4, 0.92), (0, 0.99)])
    assert OM.denoise_round(canvas, L, MASK, 0.9) == [5, 6, 2, MASK, 4]
    # nothing passes: only the most confident masked position is taken
    assert OM.denoise_round(canvas, L, MASK, 0.96) == [5, 6, 2, MASK, MASK]
    # ties: the first of the most confident
    L2 = logits_with_conf([(1, 0.3), (2, 0.6), (3, 0.6), (4, 0.6), (0, 0.99)])
    assert OM.denoise_round(canvas, L2, MASK, 0.9) == [5, 6, 2, MASK, MASK]
    # committed positions and the seed never change, even with confident predictions
    L3 = logits_with_conf([(7, 0.99), (7, 0.99), (3, 0.99), (4, 0.99), (0, 0.99)])
    assert OM.denoise_round(canvas, L3, MASK, 0.9) == [5, 6, 7, 3, 4]
    # no masks left: unchanged
    assert OM.denoise_round([5, 6, 7], L3[:3], MASK, 0.9) == [5, 6, 7]


def diffusion_model():
    cfg = HybridConfig.tiny()
    w = init_weights(cfg, seed=0, embed_scale=1.0)
    w["embed"][cfg.mask_id] = 0  # a MASK input does not predict MASK (a random model otherwise would)
    return cfg, w


def test_block_seeds_follow_causal_prefill():
    cfg, w = diffusion_model()
    m = OM.CpuHybrid(cfg, w)
    for seed in range(2):
        rng = random.Random(seed + 1)
        p = [rng.randrange(0, cfg.vocab - 10) for _ in range(20)]
        CL = 8
        out = OM.diffusion_generate(m, p, 40, canvas=CL)
        assert len(out) == 40 and cfg.mask_id not in out
        assert len(set(out)) > 3  # the loop does real work on this model
        for b in range(0, 40, CL):
            c = m.make_cache()
            ref = OM.argmax(m.prefill(c, p + out[:b]))
            assert out[b] == ref, (seed, b)
