"""Pins the GDN oracle (CPU): transformers golden fixtures, recurrent == chunked, split-carry, the
snapshot invariant and the canvas / rollback semantics of the reference runtimes."""
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as G

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return {k: torch.from_numpy(v) for k, v in np.load(GOLD / name).items()}


def rand_case(seed, B=2, T=11, Hk=2, Hv=4, Dk=32, Dv=16, unit=True):
    g0 = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hk, Dk, generator=g0)
    k = torch.randn(B, T, Hk, Dk, generator=g0)
    if unit:
        q, k = G.l2norm(q), G.l2norm(k)
    v = torch.randn(B, T, Hv, Dv, generator=g0)
    g = -F.softplus(torch.randn(B, T, Hv, generator=g0))
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=g0))
    s0 = torch.randn(B, Hv, Dv, Dk, generator=g0) * 0.1
    return q, k, v, g, beta, s0


def test_l2norm_fixture():
    d = load("l2norm_tf.npz")
    assert torch.allclose(G.l2norm(d["x"]), d["y"], atol=1e-6)


@pytest.mark.parametrize("name,fn", [("gdr_recurrent_tf.npz", "recurrent"), ("gdr_chunk_tf.npz", "chunked"),
                                     ("gdr_chunk_tf.npz", "recurrent"), ("gdr_recurrent_tf.npz", "chunked")])
def test_gdr_matches_transformers_fixture(name, fn):
    d = load(name)
    q, k = G.l2norm(d["q"]), G.l2norm(d["k"])
    o, sT = getattr(G, fn)(q, k, d["v"], d["g"], d["beta"], G.from_tf_state(d["s0"]))[:2]
    assert torch.allclose(o, d["o"], atol=2e-5, rtol=1e-4)
    assert torch.allclose(G.to_tf_state(sT), d["sT"], atol=2e-5, rtol=1e-4)


def test_gdr_fixture_catches_layout_and_gate_mistakes():
    """The fixture distinguishes the plausible mistakes: a transposed state, g used as the decay
    factor instead of its log, and a missing 1/sqrt(Dk) scale."""
    d = load("gdr_chunk_tf.npz")  # Dk == Dv, so a transposed state still has the right shape
    q, k = G.l2norm(d["q"]), G.l2norm(d["k"])
    ok = G.recurrent(q, k, d["v"], d["g"], d["beta"], G.from_tf_state(d["s0"]))[0]
    assert torch.allclose(ok, d["o"], atol=2e-5)
    bad_layout = G.recurrent(q, k, d["v"], d["g"], d["beta"], d["s0"])[0]  # not transposed
    bad_gate = G.recurrent(q, k, d["v"], torch.log(-d["g"]), d["beta"], G.from_tf_state(d["s0"]))[0]
    bad_scale = G.recurrent(q, k, d["v"], d["g"], d["beta"], G.from_tf_state(d["s0"]), scale=1.0)[0]
    for bad in (bad_layout, bad_gate, bad_scale):
        assert not torch.allclose(bad, d["o"], atol=1e-3)


def test_conv_fixture():
    d = load("conv_tf.npz")
    x = d["x"].transpose(1, 2)            # [1, T, C]
    win = d["state"].transpose(1, 2)      # [1, K-1, C]
    y, new_win = G.causal_conv(x, win, d["w"])
    assert torch.allclose(y, G.bf16_round(d["y"].transpose(1, 2)), atol=1e-2, rtol=1e-2)
    assert torch.equal(new_win, d["new_state"].transpose(1, 2))


def test_conv_closed_form():
    # a single tap on the newest row reproduces silu(w * x)
    C, K = 8, 4
    w = torch.zeros(C, K)
    w[:, -1] = 2.0
    x = torch.randn(1, 3, C)
    y, win = G.causal_conv(x, torch.randn(1, K - 1, C), w)
    assert torch.allclose(y, G.bf16_round(F.silu(2 * x)))
    assert torch.equal(win, x[:, -3:])


def test_conv_bias_matches_torch_conv1d():
    """With a bias the conv is torch's depthwise conv1d (groups = C, bias added before the SiLU) over
    [window ++ x], the layer's nn.Conv1d as the vLLM call feeds it (conv_weight, conv_bias)."""
    g0 = torch.Generator().manual_seed(11)
    B, T, C, K = 2, 5, 24, 4
    x, win = torch.randn(B, T, C, generator=g0), torch.randn(B, K - 1, C, generator=g0)
    w, bias = torch.randn(C, K, generator=g0), torch.randn(C, generator=g0)
    y, new_win = G.causal_conv(x, win, w, bias)
    full = torch.cat([win, x], 1).transpose(1, 2)                    # [B, C, K-1+T]
    ref = F.silu(F.conv1d(full, w[:, None, :], bias, groups=C)).transpose(1, 2)
    assert torch.allclose(y, G.bf16_round(ref), atol=1e-2, rtol=1e-2)
    assert torch.equal(new_win, x[:, -3:])
    # a dropped bias is caught
    y0, _ = G.causal_conv(x, win, w)
    assert not torch.allclose(y0, G.bf16_round(ref), atol=1e-2, rtol=1e-2)


def test_gates_closed_form():
    a = torch.tensor([[0.0, 30.0]])
    b = torch.tensor([[0.0, -2.0]])
    A_log = torch.log(torch.tensor([2.0, 0.5]))
    dt = torch.tensor([0.0, 0.0])
    g, beta = G.gates(a, b, A_log, dt)
    assert torch.allclose(g, torch.tensor([[-2.0 * float(np.log(2.0)), -0.5 * 30.0]]), atol=1e-6)
    assert torch.allclose(beta, torch.tensor([[0.5, 1 / (1 + float(np.exp(2.0)))]]))


def test_recurrent_matches_scalar_brute_force():
    """Dk = Dv = 1: the recurrence is scalar arithmetic, checked by hand."""
    q = torch.tensor([[[[1.0]]], [[[2.0]]]]).reshape(1, 2, 1, 1)
    k = torch.tensor([1.0, -1.0]).reshape(1, 2, 1, 1)
    v = torch.tensor([3.0, 5.0]).reshape(1, 2, 1, 1)
    g = torch.log(torch.tensor([0.5, 0.25])).reshape(1, 2, 1)
    beta = torch.tensor([0.5, 1.0]).reshape(1, 2, 1)
    s = 2.0
    outs = []
    for t in range(2):
        s = s * [0.5, 0.25][t]
        kk, qq = [1.0, -1.0][t], [1.0, 2.0][t]
        delta = ([3.0, 5.0][t] - s * kk) * [0.5, 1.0][t]
        s = s + kk * delta
        outs.append(s * qq)
    o, sT, _ = G.recurrent(q, k, v, g, beta, torch.tensor([[[[2.0]]]]), scale=1.0)
    assert torch.allclose(o.flatten(), torch.tensor(outs))
    assert abs(float(sT) - s) < 1e-6


def test_chunked_equals_recurrent_gqa():
    q, k, v, g, beta, s0 = rand_case(3, B=2, T=70, Hk=2, Hv=4)
    o1, s1, _ = G.recurrent(q, k, v, g, beta, s0)
    for C in (16, 64):
        o2, s2 = G.chunked(q, k, v, g, beta, s0, chunk=C)
        assert torch.allclose(o1, o2, atol=1e-5) and torch.allclose(s1, s2, atol=1e-5)


def test_split_carry():
    """State carried across a split equals one continuous scan (test_two_stream_cpu.py:76-84)."""
    q, k, v, g, beta, s0 = rand_case(4, T=12)
    o, s, _ = G.recurrent(q, k, v, g, beta, s0)
    oa, sa, _ = G.recurrent(q[:, :5], k[:, :5], v[:, :5], g[:, :5], beta[:, :5], s0)
    ob, sb, _ = G.recurrent(q[:, 5:], k[:, 5:], v[:, 5:], g[:, 5:], beta[:, 5:], sa)
    assert torch.allclose(torch.cat([oa, ob], 1), o, atol=1e-6) and torch.allclose(sb, s, atol=1e-6)


def test_canvas_semantics():
    q, k, v, g, beta, s0 = rand_case(5, T=7)
    snap = s0.clone()
    nc = 4
    o, s_clean, s_end = G.canvas(q, k, v, g, beta, s0, nc, causal_mode=2)
    assert torch.equal(s0, snap), "the canvas pass must not modify the entry state"
    o_ar, s_ar, states = G.recurrent(q, k, v, g, beta, s0, record_states=True)
    assert torch.equal(o[:, :nc], o_ar[:, :nc]), "clean rows are the token-causal rows"
    assert torch.allclose(s_clean, states[nc - 1]) and torch.allclose(s_end, s_ar)
    # MASK rows: block-end state read out independently (per-token loop, test_tiny.py:100-133)
    Hv, Dk = v.shape[2], k.shape[3]
    qe = q.repeat_interleave(Hv // q.shape[2], dim=2) * Dk ** -0.5
    for t in range(nc, 7):
        ref = (s_end * qe[:, t, :, None, :]).sum(-1)
        assert torch.allclose(o[:, t], ref, atol=1e-6)
    o1, _, _ = G.canvas(q, k, v, g, beta, s0, nc, causal_mode=1)
    assert torch.allclose(o1, o_ar)


def test_restore_matches_prefix_scan():
    q, k, v, g, beta, s0 = rand_case(6, B=3, T=9)
    C, K = 24, 4
    win = torch.randn(3, K - 1, C)
    pre = torch.randn(3, 9, C)
    n_keep = torch.tensor([0, 4, 9])
    st, wn = G.restore(s0, win, k, v, g, beta, pre, n_keep)
    for b, n in enumerate(n_keep.tolist()):
        ref = s0[b] if n == 0 else G.recurrent(q[b:b + 1, :n], k[b:b + 1, :n], v[b:b + 1, :n], g[b:b + 1, :n],
                                                beta[b:b + 1, :n], s0[b:b + 1])[1][0]
        assert torch.allclose(st[b], ref, atol=1e-6)
        full = torch.cat([win[b], pre[b, :n]])
        assert torch.equal(wn[b], full[-(K - 1):])


def test_prep_matches_pieces():
    B, T, Hk, Hv, Dk, Dv, K = 1, 5, 2, 4, 32, 16, 4
    C = 2 * Hk * Dk + Hv * Dv
    g0 = torch.Generator().manual_seed(7)
    x = G.bf16_round(torch.randn(B, T, C, generator=g0))
    win = G.bf16_round(torch.randn(B, K - 1, C, generator=g0))
    w = G.bf16_round(torch.randn(C, K, generator=g0) * 0.5)
    a, b = torch.randn(B, T, Hv, generator=g0), torch.randn(B, T, Hv, generator=g0)
    A_log, dt = torch.randn(Hv, generator=g0), torch.randn(Hv, generator=g0)
    q, k, v, g, beta, nw = G.prep(x, win, w, a, b, A_log, dt, Hk, Hv, Dk, Dv)
    y, _ = G.causal_conv(x, win, w)
    assert torch.allclose(q.norm(dim=-1), torch.ones(B, T, Hk), atol=1e-2)
    assert torch.equal(v.reshape(B, T, -1), y[..., 2 * Hk * Dk:])
    assert torch.equal(nw, torch.cat([win, x], 1)[:, -3:])


# ------------------------------------------------------------------ block-bidirectional readout
def _bidir_inputs(seed, B=2, T=11, Hk=2, Hv=4, Dk=8, Dv=4):
    g0 = torch.Generator().manual_seed(seed)
    q = G.l2norm(torch.randn(B, T, Hk, Dk, generator=g0))
    k = G.l2norm(torch.randn(B, T, Hk, Dk, generator=g0))
    v = torch.randn(B, T, Hv, Dv, generator=g0)
    g = -torch.nn.functional.softplus(torch.randn(B, T, Hv, generator=g0))
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=g0))
    s0 = torch.randn(B, Hv, Dv, Dk, generator=g0) * 0.1
    return q, k, v, g, beta, s0


def test_block_bidir_single_token_blocks_are_causal():
    """Blocks of one row: the reversed within-block scan from the entry state is the forward step
    itself, so the readout reduces to the causal recurrence."""
    inp = _bidir_inputs(1)
    o_ref, s_ref, _ = G.recurrent(*inp)
    o, s = G.block_bidirectional(*inp, block_size=1)
    assert torch.allclose(o, o_ref, atol=1e-6) and torch.allclose(s, s_ref, atol=1e-6)


def test_block_bidir_state_is_causal():
    inp = _bidir_inputs(2)
    _, s_ref, _ = G.recurrent(*inp)
    for bs in (2, 3, 5, 11, 64):
        _, s = G.block_bidirectional(*inp, block_size=bs)
        assert torch.allclose(s, s_ref, atol=1e-6), bs


def test_block_bidir_hand_case():
    """Scalar state (Dk = Dv = 1, k = q = 1, scale 1, no decay, beta 1/2, zero state), two rows in one
    block. Forward: o0 = v0/2, o1 = v0/4 + v1/2. Reversed from the entry state: ob1 = v1/2, ob0 =
    v0/2 + v1/4. Mean: (v0/2 + v1/8, v0/8 + v1/2)."""
    v0, v1 = 3.0, -5.0
    one = torch.ones(1, 2, 1, 1)
    v = torch.tensor([v0, v1]).reshape(1, 2, 1, 1)
    g = torch.zeros(1, 2, 1)
    beta = torch.full((1, 2, 1), 0.5)
    o, s = G.block_bidirectional(one, one, v, g, beta, torch.zeros(1, 1, 1, 1), block_size=2, scale=1.0)
    assert torch.allclose(o.flatten(), torch.tensor([v0 / 2 + v1 / 8, v0 / 8 + v1 / 2]))
    assert torch.allclose(s.flatten(), torch.tensor([v0 / 4 + v1 / 2]))
    # a second block starts from the causal state after the first (the state carried on is forward)
    v4 = torch.tensor([v0, v1, v0, v1]).reshape(1, 4, 1, 1)
    o4, _ = G.block_bidirectional(torch.ones(1, 4, 1, 1), torch.ones(1, 4, 1, 1), v4, torch.zeros(1, 4, 1),
                                  torch.full((1, 4, 1), 0.5), torch.zeros(1, 1, 1, 1), block_size=2, scale=1.0)
    assert torch.allclose(o4[0, :2].flatten(), o.flatten())
    assert not torch.allclose(o4[0, 2:].flatten(), o.flatten())
