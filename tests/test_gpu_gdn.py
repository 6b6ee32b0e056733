"""GPU parity: GDN kernels (prep, recurrent / canvas GDR, snapshot, restore) vs the CPU oracle.

Tolerances (normwise, max-abs error / max-abs reference): bf16 outputs 1e-2, fp32 states 1e-3.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as G
from trida_stack_amd import kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL_BF16 = 1e-2
TOL_F32 = 1e-3


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def gdr_inputs(seed, B, T, Hk, Hv, Dk, Dv, state_scale=0.1):
    g0 = torch.Generator().manual_seed(seed)
    q = G.bf16_round(G.l2norm(torch.randn(B, T, Hk, Dk, generator=g0)))
    k = G.bf16_round(G.l2norm(torch.randn(B, T, Hk, Dk, generator=g0)))
    v = G.bf16_round(torch.randn(B, T, Hv, Dv, generator=g0))
    g = -F.softplus(torch.randn(B, T, Hv, generator=g0))
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=g0))
    s0 = torch.randn(B, Hv, Dv, Dk, generator=g0) * state_scale
    return q, k, v, g, beta, s0


def to_dev(q, k, v, g, beta, s0):
    bf = lambda t: t.to(DEV, torch.bfloat16).contiguous()
    return bf(q), bf(k), bf(v), g.to(DEV).contiguous(), beta.to(DEV).contiguous(), s0.to(DEV).contiguous()


SHAPES = [  # (B, T, Hk, Hv, Dk, Dv)
    (2, 7, 2, 4, 32, 16),
    (1, 33, 16, 16, 128, 128),   # one verify block of the 4B-shape model
    (3, 40, 2, 4, 64, 32),       # more rows than one LDS chunk
    (2, 1, 4, 8, 128, 64),       # an AR step
    (1, 5, 1, 2, 256, 8),
]


@pytest.mark.parametrize("shape", SHAPES)
def test_gdr_recurrent_causal(gpu, shape):
    B, T, Hk, Hv, Dk, Dv = shape
    inp = gdr_inputs(sum(shape), *shape)
    o_ref, s_ref, _ = G.recurrent(*inp)
    q, k, v, g, beta, s0 = to_dev(*inp)
    s_out = torch.empty_like(s0)
    o, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=1, state_out=s_out)
    assert rel(o, o_ref) < TOL_BF16
    assert rel(s_out, s_ref) < TOL_F32
    assert torch.equal(s0.cpu(), inp[5]), "state_in must be left untouched"


@pytest.mark.parametrize("nc", [0, 1, 4, 7])
def test_gdr_canvas_block_end_readout(gpu, nc):
    shape = (2, 7, 2, 4, 32, 16)
    inp = gdr_inputs(11 + nc, *shape)
    o_ref, sc_ref, se_ref = G.canvas(*inp, num_clean=nc, causal_mode=2)
    q, k, v, g, beta, s0 = to_dev(*inp)
    s_out = torch.empty_like(s0)
    o, sc = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=2, num_clean=nc, state_out=s_out,
                                  want_clean=True)
    assert rel(o, o_ref) < TOL_BF16
    assert rel(sc, sc_ref) < TOL_F32 and rel(s_out, se_ref) < TOL_F32


def test_gdr_canvas_clean_rows_equal_causal_rows_bitwise(gpu):
    """Clean canvas rows run the same arithmetic as the token-causal pass (the lossless property)."""
    inp = gdr_inputs(21, 1, 33, 16, 16, 128, 128)
    q, k, v, g, beta, s0 = to_dev(*inp)
    o1, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=1)
    o2, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=2, num_clean=17)
    assert torch.equal(o1[:, :17], o2[:, :17])


@pytest.mark.parametrize("mode,nc", [(1, 33), (2, 1), (2, 17)])
def test_gdr_small_and_large_grid_forms_bitwise(gpu, mode, nc):
    """One sequence alone (a small grid: k and q * scale staged in fp32) and the same sequence as every
    slot of a batch of 64 (a large grid: bf16 stages) give bit-identical rows and states: both forms
    form the same products in the same order."""
    inp = gdr_inputs(31 + nc, 1, 33, 16, 16, 128, 128)
    q, k, v, g, beta, s0 = to_dev(*inp)
    rep = lambda t: t.expand(64, *t.shape[1:]).contiguous()
    s1 = torch.empty_like(s0)
    o1, c1 = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc, state_out=s1,
                                   want_clean=mode == 2)
    s64 = torch.empty_like(rep(s0))
    o64, c64 = kernels.gdr_recurrent(rep(q), rep(k), rep(v), rep(g), rep(beta), rep(s0), causal_mode=mode,
                                     num_clean=nc, state_out=s64, want_clean=mode == 2)
    for j in (0, 17, 63):
        assert torch.equal(o64[j], o1[0]) and torch.equal(s64[j], s1[0])
        if mode == 2:
            assert torch.equal(c64[j], c1[0])


def test_gdr_state_in_place(gpu):
    inp = gdr_inputs(5, 2, 9, 2, 4, 64, 32)
    _, s_ref, _ = G.recurrent(*inp)
    q, k, v, g, beta, s = to_dev(*inp)
    kernels.gdr_recurrent(q, k, v, g, beta, s, state_out=s)
    assert rel(s, s_ref) < TOL_F32


def test_gdr_prefix_4096_config2(gpu):
    """The 4096-row prefix of the benchmark config (16 heads, d=128) through the recurrent kernel."""
    inp = gdr_inputs(2, 1, 4096, 16, 16, 128, 128, state_scale=0.0)
    o_ref, s_ref, _ = G.recurrent(*inp)
    q, k, v, g, beta, s0 = to_dev(*inp)
    s_out = torch.empty_like(s0)
    o, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0, state_out=s_out)
    assert rel(o, o_ref) < TOL_BF16 and rel(s_out, s_ref) < TOL_F32


def prep_inputs(seed, B, T, Hk, Hv, Dk, Dv, Kc=4, pad=0):
    C = 2 * Hk * Dk + Hv * Dv
    g0 = torch.Generator().manual_seed(seed)
    x = G.bf16_round(torch.randn(B, T, C + pad, generator=g0))
    win = G.bf16_round(torch.randn(B, Kc - 1, C, generator=g0))
    w = G.bf16_round(torch.randn(C, Kc, generator=g0) * 0.5)
    a = G.bf16_round(torch.randn(B, T, Hv, generator=g0))
    b = G.bf16_round(torch.randn(B, T, Hv, generator=g0))
    A_log = torch.log(torch.rand(Hv, generator=g0) * 15 + 1)
    dt = torch.randn(Hv, generator=g0)
    return x, win, w, a, b, A_log, dt


@pytest.mark.parametrize("shape", [(2, 5, 2, 4, 32, 16), (1, 33, 16, 16, 128, 128), (2, 3, 2, 2, 64, 64),
                                   (1, 2, 16, 32, 128, 128),
                                   # >= 512 rows: the wide launch, one 256-thread block per row (at T = 5 most
                                   # source rows come from the window)
                                   (16, 33, 16, 16, 128, 128), (64, 9, 2, 4, 64, 32), (128, 5, 2, 4, 32, 16)])
def test_gdn_prep(gpu, shape):
    B, T, Hk, Hv, Dk, Dv = shape
    x, win, w, a, b, A_log, dt = prep_inputs(sum(shape), *shape, pad=8)
    C = w.shape[0]
    ref = G.prep(x[..., :C], win, w, a, b, A_log, dt, Hk, Hv, Dk, Dv)
    bf = lambda t: t.to(DEV, torch.bfloat16)
    wout = torch.empty(B, 3, C, dtype=torch.bfloat16, device=DEV)
    pre = torch.full((B, T, C), float("nan"), dtype=torch.bfloat16, device=DEV)
    xd = bf(x)[..., :C]  # a strided view: row stride C + 8
    got = kernels.gdn_prep(xd, bf(win), bf(w), bf(a), bf(b), A_log.to(DEV), dt.to(DEV),
                           Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, window_out=wout, pre_out=pre)
    for gt, rf, name in zip(got, ref[:5], "qkvgb"):
        assert rel(gt, rf) < TOL_BF16, name
    assert rel(got[3], ref[3]) < 1e-5 and rel(got[4], ref[4]) < 1e-5
    assert torch.equal(wout.cpu().float(), ref[5])
    assert torch.equal(pre.cpu(), xd.cpu())  # the pre-conv rows, bit for bit


def test_snapshot_restore_config2(gpu):
    """Config 2 rollback: state [16,128,128] fp32 + conv window [3, 8192] bf16; snapshot before the
    32-row block, run it (state persisted), then restore to every accepted length 0..32."""
    B, T, Hk, Hv, Dk, Dv = 1, 32, 16, 16, 128, 128
    q, k, v, g, beta, s0 = to_dev(*gdr_inputs(9, B, T, Hk, Hv, Dk, Dv))
    C = 8192
    g0 = torch.Generator().manual_seed(10)
    win0 = torch.randn(B, 3, C, generator=g0).to(DEV, torch.bfloat16)
    pre = torch.randn(B, T, C, generator=g0).to(DEV, torch.bfloat16)
    state, window = s0.clone(), win0.clone()
    snap, snap_w = torch.empty_like(state), torch.empty_like(window)
    kernels.gdn_snapshot(state, snap, window, snap_w)
    assert torch.equal(snap, state) and torch.equal(snap_w, window)
    # the block advances the live state and conv window (as a persisting pass does)
    kernels.gdr_recurrent(q, k, v, g, beta, state, state_out=state)
    window = torch.cat([window, pre], dim=1)[:, -3:].contiguous()
    for n in range(0, T + 1):
        st, wn = state.clone(), window.clone()
        kernels.gdn_restore(torch.tensor([n], dtype=torch.int32, device=DEV), snap_state=snap, state=st,
                            k=k, v=v, g=g, beta=beta, snap_window=snap_w, window=wn, preconv=pre,
                            skip_full=True)
        ref_s, ref_w = G.restore(snap.cpu(), snap_w.cpu(), k.cpu(), v.cpu(), g.cpu(), beta.cpu(), pre.cpu(),
                                 torch.tensor([n]))
        if n == T:  # skip_full: the live state already covers the whole block
            assert torch.equal(st, state)
            assert rel(st, ref_s) < TOL_F32
        else:
            assert rel(st, ref_s) < TOL_F32, n
        assert torch.equal(wn.cpu().float(), ref_w.float()), n


def test_restore_stacked_layers_in_place(gpu):
    """Layers stacked on sequences (slot b uses n_keep[b % B]); outputs alias the snapshots."""
    L, B, T, Hk, Hv, Dk, Dv, C = 3, 4, 9, 2, 4, 32, 16, 64
    inp = gdr_inputs(12, L * B, T, Hk, Hv, Dk, Dv)
    q, k, v, g, beta, s = to_dev(*inp)
    g0 = torch.Generator().manual_seed(13)
    win = torch.randn(L * B, 3, C, generator=g0).to(DEV, torch.bfloat16)
    pre = torch.randn(L * B, T, C + 8, generator=g0).to(DEV, torch.bfloat16)[..., :C]
    n_keep = torch.tensor([0, 3, 9, 5], dtype=torch.int32)
    ref_s, ref_w = G.restore(s.cpu(), win.cpu(), k.cpu(), v.cpu(), g.cpu(), beta.cpu(), pre.cpu(),
                             n_keep.repeat(L))
    kernels.gdn_restore(n_keep.to(DEV), snap_state=s, state=s, k=k, v=v, g=g, beta=beta, snap_window=win,
                        window=win, preconv=pre)
    assert rel(s, ref_s) < TOL_F32
    assert torch.equal(win.cpu().float(), ref_w.float())


@pytest.mark.parametrize("bs,shape", [(1, (2, 7, 2, 4, 32, 16)), (8, (1, 33, 16, 16, 128, 128)),
                                      (5, (3, 40, 2, 4, 64, 32)), (32, (1, 70, 2, 2, 128, 64)),
                                      (64, (1, 130, 2, 2, 64, 32))])
def test_gdr_block_bidir(gpu, bs, shape):
    """Block-bidirectional readout (train/models/hybrid.py:461-536) vs the oracle; the carried state is
    the causal one."""
    inp = gdr_inputs(60 + bs, *shape)
    o_ref, s_ref = G.block_bidirectional(*inp, block_size=bs)
    q, k, v, g, beta, s0 = to_dev(*inp)
    s_out = torch.empty_like(s0)
    o = kernels.gdr_block_bidir(q, k, v, g, beta, s0, block_size=bs, state_out=s_out)
    assert rel(o, o_ref) < TOL_BF16, rel(o, o_ref)
    assert rel(s_out, s_ref) < TOL_F32
