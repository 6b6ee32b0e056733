"""GPU parity: greedy acceptance fused into the LM head (trida_wsgemm_argmax + trida_greedy_accept_splits), and
a denoise pass's argmax / confidence readout fused into it (trida_wsgemm_argmax_conf + trida_argmax_conf_splits).

The greedy branch of _selfspec_step (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:906-914)
takes the argmax of the verify logits; here the LM-head GEMM reduces its bf16 logits to per-split (max,
first index) pairs in its epilogue, and the acceptance runs from those pairs. Bit-exact against the CPU
oracle (oracle.accept.greedy_accept) on the bf16 logits the store epilogue writes, including exact ties
across column splits and NaN rows; and the draft-then-verify and canvas steps of a model give the same
tokens, accepted lengths and committed state with and without the fused head. The readout's argmax is
row_argmax's on those logits bit for bit, its confidence (the softmax probability of the argmax, computed in
another fp32 summation order) within 1e-5, and the fp32 softmax of the logits within 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import accept as A
from trida_stack_amd import kernels
from trida_stack_amd.decode import BlockSpecStep, CanvasSpecStep
from trida_stack_amd.model import HybridConfig, build_runtime

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def head_inputs(seed, M, V, K):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * 0.5).bfloat16()
    w = (torch.randn(V, K, generator=g) * 0.05).bfloat16()
    return x, w


def run_head(x, w, want_logits=True):
    V, K = w.shape
    M = x.shape[0]
    wp = kernels.ws_shuffle(w.to(DEV).contiguous())
    S = kernels.ws_argmax_splits(V, K)
    pv = torch.empty(M * S, dtype=torch.float32, device=DEV)
    pi = torch.empty(M * S, dtype=torch.int32, device=DEV)
    lg = torch.full((M, V), float("nan"), dtype=torch.bfloat16, device=DEV) if want_logits else None
    kernels.ws_gemm_argmax(x.to(DEV).contiguous(), wp, V, pv, pi, logits=lg)
    ref = torch.empty(M, V, dtype=torch.bfloat16, device=DEV)
    kernels.ws_gemm(x.to(DEV).contiguous(), wp, V, ref)
    return pv, pi, S, lg, ref


@pytest.mark.parametrize("M,V", [(1, 4096), (7, 1040), (33, 248320), (48, 151936)])
def test_head_argmax_matches_store_epilogue(gpu, M, V):
    """The fused pairs reduce to the argmax of exactly the logits the store epilogue writes (first index
    on ties), and the optional logits output is bitwise that epilogue's."""
    x, w = head_inputs(M + V, M, V, 2560)
    # exact ties across splits: two identical weight rows, made the largest logit of token row 0
    hot = (x[0].float() / x[0].float().norm() * 8.0).bfloat16()
    lo_id, hi_id = 5, V - 7
    w[lo_id] = hot
    w[hi_id] = hot
    pv, pi, S, lg, ref = run_head(x, w)
    assert torch.equal(lg.cpu(), ref.cpu())
    drafts = torch.zeros(1, M - 1, dtype=torch.int64, device=DEV)
    am, n_acc, bonus, crop = kernels.greedy_accept_splits(pv, pi, drafts, R=M)
    want = A.greedy_accept(ref.float().cpu().numpy()[None], drafts.cpu().numpy())
    assert np.array_equal(am.cpu().numpy(), want[0])
    assert int(am[0, 0]) == lo_id  # the tie goes to the first index, across splits
    assert n_acc.cpu().tolist() == want[1].tolist() and bonus.cpu().tolist() == want[2].tolist()


def test_head_argmax_nan_rows_and_acceptance(gpu):
    """NaN logits rank above every number (the first NaN wins, as torch.argmax); drafts built from the
    argmax accept up to a planted mismatch; the crop counts ctx + 1 + n_acc."""
    M, V, K = 33, 8192, 2560
    x, w = head_inputs(3, M, V, K)
    w[1234, 7] = float("nan")
    w[4000, 9] = float("nan")
    x[5] = 0  # a row of zero logits except the NaNs: NaN * 0 is NaN, so rows 1234 and 4000 are NaN for all
    pv, pi, S, lg, ref = run_head(x, w)
    logits = ref.float().cpu().numpy()[None]
    am_ref = A.argmax_first(logits[0])
    drafts = torch.tensor(am_ref[None, :M - 1], dtype=torch.int64)
    drafts[0, 9] = (drafts[0, 9] + 1) % V  # reject at draft 9
    ctx = torch.tensor([4096], dtype=torch.int64)
    am, n_acc, bonus, crop = kernels.greedy_accept_splits(pv, pi, drafts.to(DEV), R=M, ctx_len=ctx.to(DEV))
    want = A.greedy_accept(logits, drafts.numpy(), ctx_len=ctx.numpy())
    assert np.array_equal(am.cpu().numpy(), want[0]) and int(am[0, 0]) == 1234
    assert n_acc.cpu().tolist() == want[1].tolist() == [9]
    assert bonus.cpu().tolist() == want[2].tolist() and crop.cpu().tolist() == want[3].tolist() == [4106]


@pytest.mark.parametrize("M,V", [(1, 4096), (7, 1040), (32, 248320), (48, 151936)])
def test_head_argmax_conf_matches_row_argmax(gpu, M, V):
    """The fused readout equals row_argmax on the logits the store epilogue writes: the argmax bitwise (ties
    across splits to the first index, an all-NaN row to column 0 with confidence 0), the confidence within
    1e-5, and both agree with an fp32 softmax of those logits."""
    K = 2560
    x, w = head_inputs(M * 7 + V, M, V, K)
    hot = (x[0].float() / x[0].float().norm() * 8.0).bfloat16()
    w[5] = hot
    w[V - 7] = hot
    if M > 3:
        x[3, 11] = float("nan")  # row 3: every logit NaN, its argmax column 0
    xd = x.to(DEV).contiguous()
    wp = kernels.ws_shuffle(w.to(DEV).contiguous())
    S = kernels.ws_argmax_splits(V, K)
    assert S <= kernels.CONF_MAX_SPLITS
    pv = torch.empty(M * S, dtype=torch.float32, device=DEV)
    pi = torch.empty(M * S, dtype=torch.int32, device=DEV)
    ps = torch.empty(M * S, dtype=torch.float32, device=DEV)
    kernels.ws_gemm_argmax_conf(xd, wp, V, pv, pi, ps)
    am = torch.full((1, M + 1), -1, dtype=torch.int64, device=DEV)  # row stride M + 1, as a canvas buffer
    cf = torch.full((1, M + 1), -1.0, dtype=torch.float32, device=DEV)
    kernels.argmax_conf_splits(pv, pi, ps, B=1, R=M, out=(am, cf))
    logits = torch.empty(M, V, dtype=torch.bfloat16, device=DEV)
    kernels.ws_gemm(xd, wp, V, logits)
    am_ref, cf_ref = kernels.row_argmax(logits)
    assert torch.equal(am[0, :M], am_ref) and int(am[0, M]) == -1 and float(cf[0, M]) == -1.0
    assert int(am[0, 0]) == 5
    if M > 3:
        assert int(am[0, 3]) == 0 and float(cf[0, 3]) == float(cf_ref[3]) == 0.0
    assert torch.allclose(cf[0, :M], cf_ref, rtol=1e-5, atol=0)
    lf = logits.float()
    ok = ~torch.isnan(lf).any(1)
    p_ref = torch.softmax(lf[ok], dim=1).gather(1, am_ref[ok, None])[:, 0]
    assert torch.allclose(cf[0, :M][ok], p_ref, rtol=1e-4, atol=1e-7)


@pytest.fixture(scope="module")
def rt_small(gpu):
    cfg = HybridConfig.tiny(vocab=4096)
    return build_runtime(cfg, seed=3, device=gpu)


def _twin_caches(rt, prompt, T):
    out = []
    for _ in range(2):
        c = rt.make_cache(1, max_len=len(prompt) + 8 * T + 64)
        rt.prefill(c, prompt)
        out.append(c)
    return out


@pytest.mark.parametrize("flag", ["fused_greedy_head", "fused_draft_head"])
def test_blockspec_step_fused_head_equals_unfused(gpu, rt_small, flag):
    """Draft-then-verify steps (block 16, 2 denoising passes) with the fused heads (the denoise readout and
    the greedy acceptance) and with one of them (or, without the greedy head, both) on logits + row_argmax /
    trida_greedy_accept: identical drafts, argmax rows, accepted lengths, bonus tokens and committed caches,
    step after step."""
    rt = rt_small
    assert rt.greedy_head_ok(17) and rt.argmax_conf_ok()
    g = torch.Generator().manual_seed(9)
    prompt = torch.randint(0, rt.cfg.vocab - 2, (50,), generator=g).tolist()
    ca, cb = _twin_caches(rt, prompt, 17)
    sa, sb = BlockSpecStep(rt, ca, 16, 2), BlockSpecStep(rt, cb, 16, 2)
    sa.t0.fill_(7)
    sb.t0.fill_(7)
    for _ in range(4):
        sa.run()
        setattr(rt, flag, False)
        try:
            sb.run()
        finally:
            setattr(rt, flag, True)
        for name in ("canvas", "am", "n_acc", "bonus", "crop"):
            assert torch.equal(getattr(sa, name), getattr(sb, name)), name
        assert torch.equal(ca.length, cb.length)
        assert torch.equal(ca.state, cb.state) and torch.equal(ca.window, cb.window)


def test_canvas_step_fused_head_equals_unfused(gpu, rt_small):
    """The canvas algorithm (N = 4, canvas of 7 rows) with and without the fused head: the same emitted
    and committed tokens and caches."""
    rt = rt_small
    g = torch.Generator().manual_seed(10)
    prompt = torch.randint(0, rt.cfg.vocab - 2, (40,), generator=g).tolist()
    ca, cb = _twin_caches(rt, prompt, 7)
    sa, sb = CanvasSpecStep(rt, ca, 4), CanvasSpecStep(rt, cb, 4)
    t0 = torch.tensor([11], dtype=torch.int64, device=DEV)
    sa.start(t0)
    sb.start(t0)
    for _ in range(5):
        sa.run()
        rt.fused_greedy_head = False
        try:
            sb.run()
        finally:
            rt.fused_greedy_head = True
        for name in ("canvas", "am", "emit", "n_emit", "committed", "n_keep", "kind"):
            assert torch.equal(getattr(sa, name), getattr(sb, name)), name
        assert torch.equal(ca.state, cb.state) and torch.equal(ca.length, cb.length)
