"""GPU parity: a GDN layer's gated RMSNorm folded into its recurrence and out projection
(trida_gdr_recurrent_gnorm + trida_wsgemm_headnorm) against the unfolded kernels (trida_gdr_recurrent,
trida_gated_rmsnorm_frag, trida_wsgemm_ex epilogue 1) and an fp32 torch restatement of the layer's tail,
y = rmsnorm(o) * w * silu(z) per value head, out = y W^T (the reference's RMSNormGated then out_proj,
inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:2207-2221).

The recurrence output o and the states are bitwise those of trida_gdr_recurrent; the projection differs from
the unfolded one only in where the bf16 roundings fall (the fold never forms bf16(o * inv)): within 1e-2
normwise of both the unfolded kernels and the fp32 restatement.
"""
import pytest
import torch

from trida_stack_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def inputs(seed, B, T, Hk, Hv, Dk, Dv, N):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, Hk, Dk, generator=g), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(B, T, Hk, Dk, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, T, Hv, Dv, generator=g).bfloat16()
    gl = -torch.rand(B, T, Hv, generator=g) * 0.5
    beta = torch.rand(B, T, Hv, generator=g)
    state = torch.randn(B, Hv, Dv, Dk, generator=g) * 0.1
    z = torch.randn(B * T, 2 * Hv * Dv + 8, generator=g).bfloat16()  # wider rows: z is a slice of the in-proj
    w = (1.0 + 0.3 * torch.randn(Dv, generator=g)).bfloat16()
    wout = (torch.randn(N, Hv * Dv, generator=g) * 0.03).bfloat16()
    return [t.to(DEV) for t in (q, k, v, gl, beta, state, z, w, wout)]


@pytest.mark.parametrize("B,T,Hk,Hv,Dk,Dv,N,mode", [
    (1, 33, 16, 16, 128, 128, 2560, 1),   # the 4B-shape verify block
    (1, 33, 16, 16, 128, 128, 2560, 2),   # a denoising pass (rows >= 1 read the block-end state)
    (1, 1, 16, 16, 128, 128, 2560, 1),    # one AR row
    (1, 17, 2, 4, 32, 64, 128, 2),        # the tiny test model's GDN geometry
    (2, 20, 4, 8, 64, 128, 512, 1),       # two sequences, 40 rows
])
def test_gnorm_fold_matches_unfolded(gpu, B, T, Hk, Hv, Dk, Dv, N, mode):
    q, k, v, gl, beta, state, zfull, w, wout = inputs(B * 100 + T + Dv + mode, B, T, Hk, Hv, Dk, Dv, N)
    z = zfull[:, Hv * Dv: 2 * Hv * Dv]  # a strided slice, as the forward takes it from the in-projection rows
    nc = 1 if mode == 2 else T
    M, VD = B * T, Hv * Dv
    eps = 1e-6
    # unfolded: recurrence, gated norm into fragment order, partial-plane projection
    s_a = state.clone()
    o_a, _ = K.gdr_recurrent(q, k, v, gl, beta, state, causal_mode=mode, num_clean=nc, state_out=s_a)
    yf = torch.empty(K.ws_frag_numel(VD), dtype=torch.bfloat16, device=DEV)
    K.gated_rmsnorm(o_a.view(M, Hv, Dv), z, w, yf, eps=eps, out_frag=True)
    wp = K.ws_shuffle(wout.contiguous())
    kg_a = K.ws_plan(N, VD, K.WS_PARTS)
    parts_a = torch.empty(kg_a * M * N, dtype=torch.float32, device=DEV)
    K.ws_gemm_frag(yf, M, wp, N, parts_a, epilogue=K.WS_PARTS)
    out_a = parts_a.view(kg_a, M, N).sum(0)
    # folded
    s_b = state.clone()
    uf = torch.zeros(K.ws_frag_numel(VD), dtype=torch.bfloat16, device=DEV)
    ss = torch.full((M * Hv * (Dv // 8),), float("nan"), dtype=torch.float32, device=DEV)
    o_b = K.gdr_recurrent_gnorm(q, k, v, gl, beta, state, z, w, uf, ss, causal_mode=mode, num_clean=nc,
                                state_out=s_b)
    kg_b = K.ws_headnorm_planes(N, VD, Hv)
    parts_b = torch.full((kg_b * M * N,), float("nan"), dtype=torch.float32, device=DEV)
    assert K.ws_gemm_headnorm(uf, M, wp, N, ss, Hv, parts_b, eps=eps) == kg_b
    out_b = parts_b.view(kg_b, M, N).sum(0)
    # the recurrence itself is unchanged
    assert torch.equal(o_a, o_b) and torch.equal(s_a, s_b)
    # the sums of squares: bf16(o)^2 over each 8 columns
    of = o_a.float().view(M, Hv, Dv // 8, 8)
    assert torch.allclose(ss.view(M, Hv, Dv // 8), (of * of).sum(-1), rtol=1e-5, atol=1e-6)
    # fp32 restatement of the layer's tail
    o32 = o_a.float().view(M, Hv, Dv)
    inv = torch.rsqrt(o32.pow(2).mean(-1, keepdim=True) + eps)
    y = (o32 * inv) * w.float() * torch.nn.functional.silu(z.float().view(M, Hv, Dv))
    ref = y.view(M, VD) @ wout.float().t()
    assert torch.isfinite(out_b).all()
    assert rel(out_b, ref) < 1e-2, rel(out_b, ref)
    assert rel(out_b, out_a) < 1e-2, rel(out_b, out_a)


def test_gnorm_fold_rejects_long_blocks(gpu):
    """More rows than one staged chunk (or than the fragment order holds) are refused, not mis-computed."""
    B, T, Hk, Hv, Dk, Dv, N = 1, 41, 2, 4, 32, 64, 128
    q, k, v, gl, beta, state, zfull, w, wout = inputs(5, B, T, Hk, Hv, Dk, Dv, N)
    z = zfull[:, : Hv * Dv]
    uf = torch.zeros(K.ws_frag_numel(Hv * Dv), dtype=torch.bfloat16, device=DEV)
    ss = torch.zeros(B * T * Hv * (Dv // 8), dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="T <= 40"):
        K.gdr_recurrent_gnorm(q, k, v, gl, beta, state, z, w, uf, ss)
