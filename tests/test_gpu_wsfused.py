"""GPU parity of the fused decode-step path: the residual add over partial planes (residual_parts), the
weight-streaming GEMM with the RMSNorm prologue (ws_gemm_norm), and a small model whose every projection
runs on them, against torch references and the CPU oracle."""
import random

import pytest
import torch
import torch.nn.functional as F

from oracle import model as OM
from trida_stack_amd import kernels as TK
from trida_stack_amd.decode import SamplingParams, ar_generate, selfspec_generate
from trida_stack_amd.model import HybridConfig, TridaRuntime, init_weights

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
# every projection shape divisible for the weight-streaming GEMM (N % 16, K % 32), hidden <= 2560
CFG = HybridConfig(hidden=256, n_layers=4, intermediate=512, vocab=300, lin_k_heads=2, lin_v_heads=8, lin_k_dim=32,
                   lin_v_dim=64, n_heads=4, n_kv_heads=2, head_dim=64, rope_theta=10000.0, mask_id=299)


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def bf(x):
    return x.to(torch.bfloat16).float()


@pytest.mark.parametrize("dim,n_parts", [(2560, 0), (2560, 1), (2560, 8), (128, 3), (260, 2)])
def test_residual_parts(gpu, dim, n_parts):
    g = torch.Generator().manual_seed(dim + n_parts)
    rows = 33
    h = torch.randn(rows, dim, generator=g).to(torch.bfloat16)
    parts = torch.randn(max(n_parts, 1), rows, dim, generator=g) * 0.3
    acc = torch.zeros(rows, dim)
    for s in range(n_parts):
        acc += parts[s]
    h_ref = bf(h.float() + bf(acc)) if n_parts else h.float()
    C = TK.ss_chunks(dim)
    assert C == -(-dim // 256)
    ss_ref = torch.stack([(h_ref[:, c * 256:(c + 1) * 256] ** 2).sum(1) for c in range(C)], 1)
    hd, ss = h.to(DEV), torch.full((rows, C), float("nan"), device=DEV)
    TK.residual_parts(hd, parts.to(DEV) if n_parts else None, n_parts, ss)
    assert torch.equal(hd.float().cpu(), h_ref)  # the bf16 residual stream, bit for bit
    assert rel(ss, ss_ref) < 1e-5


@pytest.mark.parametrize("M,N,K,epi", [(33, 8224, 2560, 0), (1, 10240, 2560, 0), (33, 19456, 2560, 2),
                                       (17, 64, 256, 0), (5, 128, 96, 2)])
def test_ws_gemm_norm(gpu, M, N, K, epi):
    """rmsnorm(h) * (1 + w) @ W^T with the norm weight folded into the shuffled weights' columns and the
    row scale rsqrt(mean(h^2) + eps) applied in the epilogue."""
    g = torch.Generator().manual_seed(M + N + K)
    h = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    nw = (torch.randn(K, generator=g) * 0.1).to(torch.bfloat16)
    hd = h.to(DEV)
    ss = torch.empty(M, TK.ss_chunks(K), device=DEV)
    TK.residual_parts(hd, None, 0, ss)
    inv = torch.rsqrt(h.float().pow(2).mean(1) + 1e-6)
    y = (h.float() * inv[:, None] * (1.0 + nw.float())) @ w.float().t()  # the operator, in fp32
    if epi == TK.WS_SILU:
        y = bf(y)
        y = F.silu(y[:, : N // 2]) * y[:, N // 2:]
    wp = TK.ws_shuffle(w.to(DEV), pair_halves=epi == TK.WS_SILU, col_scale=nw.to(DEV))
    # the folded copy: bf16(w * (1 + nw)) column by column
    plain = TK.ws_shuffle(bf(w.float() * (1.0 + nw.float())).to(torch.bfloat16).to(DEV), pair_halves=epi == TK.WS_SILU)
    assert torch.equal(wp, plain)
    out = torch.empty(M, N // 2 if epi == TK.WS_SILU else N, dtype=torch.bfloat16, device=DEV)
    TK.ws_gemm_norm(hd, ss, wp, N, out, epilogue=epi)
    assert rel(out, y) < 2e-2
    # the same rows for any M (row 0 alone)
    out1 = torch.empty(1, out.shape[1], dtype=torch.bfloat16, device=DEV)
    TK.ws_gemm_norm(hd[:1], ss[:1], wp, N, out1, epilogue=epi)
    assert torch.equal(out1, out[:1])


@pytest.mark.parametrize("M,N,K,epi,norm", [(33, 8224, 2560, 0, True), (33, 19456, 2560, 2, True),
                                            (33, 2560, 9728, 1, False), (1, 2560, 2048, 1, False),
                                            (48, 256, 96, 2, False), (17, 128, 256, 0, False), (5, 64, 320, 2, True)])
def test_ws_gemm_fragment_order(gpu, M, N, K, epi, norm):
    """X in fragment order (converted, or written by the producers the fused forward uses) gives bitwise
    the row-major GEMM's result, and a fragment-order output is bitwise the row-major output converted."""
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    wp = TK.ws_shuffle(w, pair_halves=epi == TK.WS_SILU)
    xf = TK.ws_frag(x)
    ss = None
    if norm:
        ss = torch.empty(M, TK.ss_chunks(K), device=DEV)
        hf = torch.full((TK.ws_frag_numel(K),), float("nan"), dtype=torch.bfloat16, device=DEV)
        TK.residual_parts(x, None, 0, ss, h_frag=hf)  # the residual kernel's own copy of h
        mask = _frag_mask(M, K)
        assert torch.equal(hf.view(torch.int16).cpu()[mask], xf.view(torch.int16).cpu()[mask])
    width = N // 2 if epi == TK.WS_SILU else N
    if epi == TK.WS_PARTS:
        kg = TK.ws_plan(N, K, epi)
        ref = torch.empty(kg * M * N, device=DEV)
        got = torch.full_like(ref, float("nan"))
        TK.ws_gemm(x, wp, N, ref, epilogue=epi)
        TK.ws_gemm_frag(xf, M, wp, N, got, epilogue=epi)
        assert torch.equal(got, ref)
        return
    ref = torch.empty(M, width, dtype=torch.bfloat16, device=DEV)
    if norm:
        TK.ws_gemm_norm(x, ss, wp, N, ref, epilogue=epi)
    else:
        TK.ws_gemm(x, wp, N, ref, epilogue=epi)
    got = torch.empty_like(ref)
    TK.ws_gemm_frag(xf, M, wp, N, got, ss=ss, epilogue=epi)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    if width % 32 == 0:
        of = torch.zeros(TK.ws_frag_numel(width), dtype=torch.bfloat16, device=DEV)
        TK.ws_gemm_frag(xf, M, wp, N, of, ss=ss, epilogue=epi, out_frag=True)
        mask = _frag_mask(M, width)
        assert torch.equal(of.view(torch.int16).cpu()[mask], TK.ws_frag(ref).view(torch.int16).cpu()[mask])


def _frag_mask(M, K):
    """The fragment-order entries of rows < M (the rest is never written nor read)."""
    import numpy as np
    m, k = np.meshgrid(np.arange(M), np.arange(K), indexing="ij")
    off = (((k // 32) * 3 + m // 16) * 64 + ((k % 32) // 8) * 16 + m % 16) * 8 + k % 8
    mask = torch.zeros(K // 32 * 3 * 64 * 8, dtype=torch.bool)
    mask[torch.from_numpy(off.ravel())] = True
    return mask


@pytest.mark.parametrize("rows,H,Dv", [(33, 16, 128), (7, 4, 256), (48, 2, 64)])
def test_gated_rmsnorm_fragment_order(gpu, rows, H, Dv):
    g = torch.Generator().manual_seed(rows + H + Dv)
    o = torch.randn(rows, H, Dv, generator=g).to(torch.bfloat16).to(DEV)
    z = torch.randn(rows, H * Dv + 64, generator=g).to(torch.bfloat16).to(DEV)[:, 32: 32 + H * Dv]
    w = (torch.randn(Dv, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    ref = torch.empty(rows, H, Dv, dtype=torch.bfloat16, device=DEV)
    TK.gated_rmsnorm(o, z, w, ref)
    of = torch.zeros(TK.ws_frag_numel(H * Dv), dtype=torch.bfloat16, device=DEV)
    TK.gated_rmsnorm(o, z, w, of, out_frag=True)
    mask = _frag_mask(rows, H * Dv)
    assert torch.equal(of.view(torch.int16).cpu()[mask], TK.ws_frag(ref.view(rows, -1)).view(torch.int16).cpu()[mask])


def test_attn_canvas_fragment_order(gpu):
    """The attention output written in fragment order is bitwise the row-major output converted."""
    g = torch.Generator().manual_seed(3)
    B, T, Hq, Hkv, D, L = 1, 33, 16, 4, 256, 200
    q = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16).to(DEV)
    gate = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    pl = torch.tensor([120], dtype=torch.int32, device=DEV)
    ref = TK.attn_canvas(q, kc, vc, pl, mask_mode=TK.MASK_VERIFY, gate=gate)
    of = torch.zeros(TK.ws_frag_numel(Hq * D), dtype=torch.bfloat16, device=DEV)
    TK.attn_canvas(q, kc, vc, pl, mask_mode=TK.MASK_VERIFY, gate=gate, out=of, out_frag=True)
    mask = _frag_mask(B * T, Hq * D)
    assert torch.equal(of.view(torch.int16).cpu()[mask],
                       TK.ws_frag(ref.view(B * T, -1)).view(torch.int16).cpu()[mask])


@pytest.fixture(scope="module")
def fused_pair():
    w = init_weights(CFG, seed=0, embed_scale=4.0)
    rt = TridaRuntime(CFG, w, device=DEV)
    assert rt.ws_fused, "the test config must run every projection on the weight-streaming GEMM"
    return rt, OM.CpuHybrid(CFG, w)


def prompt(n, seed=1):
    rng = random.Random(seed)
    return [rng.randrange(0, CFG.vocab - 10) for _ in range(n)]


def test_fused_forward_matches_oracle(gpu, fused_pair):
    rt, m = fused_pair
    p = prompt(29)
    c, co = rt.make_cache(max_len=160), m.make_cache()
    assert rel(rt.prefill(c, p), m.prefill(co, p)) < 2e-2
    n = 16  # a canvas of 31 rows: the fused path (<= 48 rows)
    canvas = prompt(n, seed=5) + [CFG.mask_id] * (n - 1)
    for mode in ("canvas", "draft", "verify"):
        g = rt.forward(torch.tensor([canvas], device=DEV), c, mode, n_clean=n)[0]
        o = m.forward(canvas, co, mode, n_clean=n)
        co.pending = None
        assert rel(g, o) < 2e-2, mode


def test_fused_forward_matches_unfused(gpu, fused_pair):
    """The same weights through add_rmsnorm + hipBLASLt projections (use_wsgemm off)."""
    rt, _ = fused_pair
    old = TridaRuntime.use_wsgemm
    try:
        TridaRuntime.use_wsgemm = False
        ref = TridaRuntime(CFG, {k: v.cpu() for k, v in rt.w.items()}, device=DEV)
    finally:
        TridaRuntime.use_wsgemm = old
    assert not ref.ws and not ref.ws_fused
    p = prompt(40, seed=3)
    ca, cb = rt.make_cache(max_len=128), ref.make_cache(max_len=128)
    rt.prefill(ca, p)
    ref.prefill(cb, p)
    ids = torch.tensor([prompt(33, seed=9)], device=DEV)
    assert rel(rt.forward(ids, ca, "verify"), ref.forward(ids, cb, "verify")) < 2e-2


def collect(gen):
    out = []
    for ch in gen:
        out.extend(ch)
    return out


def test_fused_greedy_selfspec_equals_ar(gpu, fused_pair):
    """Lossless greedy self-spec on the fused path: the same tokens as greedy AR under the token-recurrent
    GDN form (AR rows run the projections with M = 1, canvas rows with M = 7 or 16; the projections are
    bitwise independent of M)."""
    rt, _ = fused_pair
    old = rt.gdr_form
    rt.gdr_form = "recurrent"
    try:
        sp = SamplingParams(temperature=0.0)
        for seed in range(2):
            p = prompt(25, seed=seed + 10)
            ar = collect(ar_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=48, eos_ids=set(), sp=sp))
            ss = collect(selfspec_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=48, eos_ids=set(),
                                           sp=sp, mask_id=CFG.mask_id, n=4))
            bs = collect(selfspec_generate(rt, rt.make_cache(max_len=256), p, max_new_tokens=48, eos_ids=set(),
                                           sp=sp, mask_id=CFG.mask_id, n=8, denoise_steps=2))
            assert ss == ar, f"seed {seed}"
            assert bs == ar, f"seed {seed} block"
    finally:
        rt.gdr_form = old
