"""GPU parity: the fused GDN layer (conv + prep + recurrence + readout in one launch) against the
two-launch path (trida_gdn_prep then trida_gdr_recurrent), bit for bit, and against the CPU oracle.

The two-launch path is itself pinned to the oracle (tests/test_gpu_gdn.py), so bit-equality carries its
parity over; one oracle comparison is kept here as an independent check (bf16 outputs 1e-2, fp32
states 1e-3, normwise).
"""
import pytest
import torch

from oracle import gdn as G
from trida_stack_amd import kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def layer_inputs(seed, B, T, Hk, Hv, Dk, Dv, Kc):
    """Pre-conv rows inside a wider projection row (as the in-projection writes them), a/b as strided
    slices of one tensor, conv window, weights and a starting state."""
    C = 2 * Hk * Dk + Hv * Dv
    g0 = torch.Generator().manual_seed(seed)
    width = (C + 2 * Hv + 7) // 8 * 8 + 8  # row stride a multiple of 8 elements, as the kernels require
    proj = G.bf16_round(torch.randn(B, T, width, generator=g0))
    win = G.bf16_round(torch.randn(B, Kc - 1, C, generator=g0))
    w = G.bf16_round(torch.randn(C, Kc, generator=g0) * 0.5)
    A_log = torch.log(torch.rand(Hv, generator=g0) * 15 + 1)
    dt = torch.randn(Hv, generator=g0)
    s0 = torch.randn(B, Hv, Dv, Dk, generator=g0) * 0.1
    return proj, win, w, A_log, dt, s0


def split(proj, C, Hv):
    return proj[..., :C], proj[..., C:C + Hv], proj[..., C + Hv:C + 2 * Hv]  # x, b, a


CASES = [  # (B, T, Hk, Hv, Dk, Dv, Kc, causal_mode, num_clean)
    (1, 33, 16, 16, 128, 128, 4, 1, None),  # verify block of the 4B-shape model (2 waves per block)
    (1, 33, 16, 16, 128, 128, 4, 2, 1),     # denoising pass
    (8, 33, 16, 16, 128, 128, 4, 1, None),  # batch 8 (4 waves per block)
    (2, 64, 2, 4, 64, 32, 3, 2, 17),        # maximum rows, GQA, 1 wave per block
    (3, 1, 4, 8, 32, 16, 2, 1, None),       # an AR step, conv width 2
    (2, 7, 1, 2, 128, 8, 4, 2, 0),          # no clean rows
]


@pytest.mark.parametrize("case", CASES)
def test_fused_layer_equals_two_launch_path(gpu, case):
    B, T, Hk, Hv, Dk, Dv, Kc, mode, nc = case
    C = 2 * Hk * Dk + Hv * Dv
    proj, win, w, A_log, dt, s0 = layer_inputs(sum(x or 0 for x in case), B, T, Hk, Hv, Dk, Dv, Kc)
    bf = lambda t: t.to(DEV, torch.bfloat16)
    projd, wind, wd, s0d = bf(proj), bf(win).contiguous(), bf(w).contiguous(), s0.to(DEV).contiguous()
    x, b_in, a_in = split(projd, C, Hv)
    A_logd, dtd = A_log.to(DEV), dt.to(DEV)

    # two launches
    wout_ref = torch.empty_like(wind)
    q, k, v, g, beta = kernels.gdn_prep(x, wind, wd, a_in, b_in, A_logd, dtd, Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv,
                                        window_out=wout_ref)
    s_ref = torch.empty_like(s0d)
    o_ref, clean_ref = kernels.gdr_recurrent(q, k, v, g, beta, s0d, causal_mode=mode, num_clean=nc,
                                             state_out=s_ref, want_clean=True)
    # one launch, every optional output requested
    rows = (torch.full_like(k, 7), torch.full_like(v, 7), torch.full_like(g, 7), torch.full_like(beta, 7))
    pre = torch.zeros(B, T, C, dtype=torch.bfloat16, device=DEV)
    wout = torch.zeros_like(wind)
    s_out = torch.empty_like(s0d)
    o, clean = kernels.gdn_fused_layer(x, wind, wd, a_in, b_in, A_logd, dtd, s0d, Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv,
                                       causal_mode=mode, num_clean=nc, state_out=s_out, want_clean=True,
                                       rows_out=rows, pre_out=pre, window_out=wout)
    assert torch.equal(o, o_ref)
    assert torch.equal(s_out, s_ref)
    assert torch.equal(clean, clean_ref)
    for got, ref, name in zip(rows, (k, v, g, beta), ("k", "v", "g", "beta")):
        assert torch.equal(got, ref), name
    assert torch.equal(pre, x.contiguous())
    assert torch.equal(wout, wout_ref)
    assert torch.equal(s0d.cpu(), s0), "state_in must be left untouched"


def test_fused_layer_optional_outputs_and_in_place_state(gpu):
    """A denoising pass writes only the readout; a persisting pass advances the state in place."""
    B, T, Hk, Hv, Dk, Dv, Kc = 1, 33, 16, 16, 128, 128, 4
    C = 2 * Hk * Dk + Hv * Dv
    proj, win, w, A_log, dt, s0 = layer_inputs(5, B, T, Hk, Hv, Dk, Dv, Kc)
    bf = lambda t: t.to(DEV, torch.bfloat16)
    projd, wind, wd = bf(proj), bf(win).contiguous(), bf(w).contiguous()
    x, b_in, a_in = split(projd, C, Hv)
    args = (x, wind, wd, a_in, b_in, A_log.to(DEV), dt.to(DEV))
    geo = dict(Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv)
    s_live = s0.to(DEV).contiguous()
    o_draft, _ = kernels.gdn_fused_layer(*args, s_live, causal_mode=2, num_clean=1, **geo)
    assert torch.equal(s_live.cpu(), s0)
    s_sep = torch.empty_like(s_live)
    o1, _ = kernels.gdn_fused_layer(*args, s_live, state_out=s_sep, **geo)
    o2, _ = kernels.gdn_fused_layer(*args, s_live, state_out=s_live, **geo)  # in place
    assert torch.equal(o1, o2) and torch.equal(s_live, s_sep)
    q, k, v, g, beta = kernels.gdn_prep(*args, **geo)
    o_ref, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0.to(DEV).contiguous(), causal_mode=2, num_clean=1)
    assert torch.equal(o_draft, o_ref)


@pytest.mark.parametrize("mode,nc", [(1, None), (2, 3)])
def test_fused_layer_vs_oracle(gpu, mode, nc):
    B, T, Hk, Hv, Dk, Dv, Kc = 2, 9, 2, 4, 64, 32, 4
    C = 2 * Hk * Dk + Hv * Dv
    proj, win, w, A_log, dt, s0 = layer_inputs(11, B, T, Hk, Hv, Dk, Dv, Kc)
    x, b_in, a_in = split(proj, C, Hv)
    q, k, v, g, beta, wnew = G.prep(x, win, w, a_in, b_in, A_log, dt, Hk, Hv, Dk, Dv)
    if mode == 1:
        o_ref, s_ref, _ = G.recurrent(q, k, v, g, beta, s0)
    else:
        o_ref, _, s_ref = G.canvas(q, k, v, g, beta, s0, num_clean=nc)
    bf = lambda t: t.to(DEV, torch.bfloat16)
    projd = bf(proj)
    xd, bd, ad = split(projd, C, Hv)
    s_out = torch.empty(B, Hv, Dv, Dk, device=DEV)
    wout = torch.empty(B, Kc - 1, C, dtype=torch.bfloat16, device=DEV)
    o, _ = kernels.gdn_fused_layer(xd, bf(win).contiguous(), bf(w).contiguous(), ad, bd, A_log.to(DEV), dt.to(DEV),
                                   s0.to(DEV).contiguous(), Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, causal_mode=mode,
                                   num_clean=nc, state_out=s_out, window_out=wout)
    assert rel(o, o_ref) < 1e-2
    assert rel(s_out, s_ref) < 1e-3
    assert torch.equal(wout.cpu().float(), wnew)


def test_fused_layer_argument_checks(gpu):
    B, T, Hk, Hv, Dk, Dv, Kc = 1, 65, 1, 1, 32, 8, 4
    C = 2 * Hk * Dk + Hv * Dv
    x = torch.zeros(B, T, C + 2 * Hv, dtype=torch.bfloat16, device=DEV)
    win = torch.zeros(B, Kc - 1, C, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(C, Kc, dtype=torch.bfloat16, device=DEV)
    ab = x[..., C:C + Hv]
    s = torch.zeros(B, Hv, Dv, Dk, device=DEV)
    one = torch.zeros(Hv, device=DEV)
    with pytest.raises(ValueError):  # more than 64 rows
        kernels.gdn_fused_layer(x[..., :C], win, w, ab, ab, one, one, s, Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv)
    with pytest.raises(ValueError):  # window_out aliasing window
        kernels.gdn_fused_layer(x[:, :4, :C], win, w, ab[:, :4], ab[:, :4], one, one, s, Hk=Hk, Hv=Hv, Dk=Dk,
                                Dv=Dv, window_out=win)
