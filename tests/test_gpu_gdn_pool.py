"""GPU parity: the GDN entry points in the layouts of the reference's vLLM calls, through the C-ABI.

The self-spec step of inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py keeps its GDN
state in pools and a two-deep ring instead of contiguous per-batch buffers:

- ring [2R+1, N, Hv, Dv, Dk] fp32 per layer (:1821-1837); a request in slot s with parity `par` and
  `pacc` drafts accepted last step reads its initial state from ring row (par R + s, pacc) and writes
  the states after rows 0..N-1 of its canvas to ring row (1 - par) R + s (_ss_index_prep_kernel,
  :228-248);
- conv windows [R+2, Kc-1, C], row s + 1 (row 0 is vLLM's null block); pre-conv rows [R+1, blk, C],
  slot s; conv_bias of the layer's conv1d (fused_selfspec_gdn_layer, :2211-2220);
- prefill batches packed as ragged sequences with cu_seqlens (:2408-2415).

Each case runs a permuted slot map and is compared with the CPU oracle per request: outputs within
1e-2 and every written state within 1e-3 (normwise), pre-conv rows and untouched pool rows bit for bit.
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


def bf(t):
    return t.to(DEV, torch.bfloat16).contiguous()


def i32(xs):
    return torch.tensor(xs, dtype=torch.int32, device=DEV)


def layer_weights(g0, Hk, Hv, Dk, Dv, Kc=4):
    C = 2 * Hk * Dk + Hv * Dv
    conv_w = G.bf16_round(torch.randn(C, Kc, generator=g0) * 0.5)
    conv_b = G.bf16_round(torch.randn(C, generator=g0) * 0.2)
    A_log = torch.randn(Hv, generator=g0) * 0.5
    dt = torch.randn(Hv, generator=g0)
    return C, conv_w, conv_b, A_log, dt


@pytest.mark.parametrize("geo", [(2, 4, 32, 16), (16, 16, 128, 128)])
def test_fused_layer_selfspec_ring(gpu, geo):
    """fused_selfspec_gdn_layer(..., conv_bias, win, win_idx, ssm_states=ring[prev], ssm_idx, inter=ring[cur],
    inter_idx, num_clean=N, cache_steps=N, pre_out, slot_idx) with three requests in permuted slots."""
    Hk, Hv, Dk, Dv = geo
    g0 = torch.Generator().manual_seed(Hk * 7 + Dk)
    R, N = 5, 4
    blk = 2 * N - 1
    C, conv_w, conv_b, A_log, dt = layer_weights(g0, Hk, Hv, Dk, Dv)
    slots, par, pacc = [3, 0, 4], [0, 1, 0], [2, 0, 3]
    n = len(slots)
    ssm_idx = [(p * R + s) * N + a for s, p, a in zip(slots, par, pacc)]
    write_idx = [(1 - p) * R + s for s, p in zip(slots, par)]
    ring = torch.randn(2 * R + 1, N, Hv, Dv, Dk, generator=g0) * 0.1
    win_pool = G.bf16_round(torch.randn(R + 2, 3, C, generator=g0))
    pre_pool = torch.zeros(R + 1, blk, C)
    x = G.bf16_round(torch.randn(n, blk, C, generator=g0))
    a_in = G.bf16_round(torch.randn(n, blk, Hv, generator=g0))
    b_in = G.bf16_round(torch.randn(n, blk, Hv, generator=g0))

    ring_d = ring.to(DEV).contiguous()
    pre_d = bf(pre_pool)
    out, _ = kernels.gdn_fused_layer(
        bf(x), bf(win_pool), bf(conv_w), bf(a_in), bf(b_in), A_log.to(DEV), dt.to(DEV),
        ring_d.view((2 * R + 1) * N, Hv, Dv, Dk), Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, causal_mode=2, num_clean=N,
        pre_out=pre_d, conv_bias=bf(conv_b), win_idx=i32([s + 1 for s in slots]), state_idx=i32(ssm_idx),
        inter=ring_d, inter_idx=i32(write_idx), cache_steps=N, pre_idx=i32(slots))
    torch.cuda.synchronize()
    ring_got, pre_got = ring_d.cpu(), pre_d.cpu()
    written = set()
    for i, s in enumerate(slots):
        q, k, v, g, beta, _ = G.prep(x[i:i + 1], win_pool[s + 1:s + 2], conv_w, a_in[i:i + 1], b_in[i:i + 1], A_log,
                                     dt, Hk, Hv, Dk, Dv, conv_bias=conv_b)
        s0 = ring[par[i] * R + s, pacc[i]][None]
        o_ref, _, _ = G.canvas(q, k, v, g, beta, s0, num_clean=N, causal_mode=2)
        _, _, states = G.recurrent(q, k, v, g, beta, s0, record_states=True)
        assert rel(out[i], o_ref[0]) < TOL_BF16, f"request {i} readout"
        for j in range(N):
            assert rel(ring_got[write_idx[i], j], states[j][0]) < TOL_F32, f"request {i} ring state after row {j}"
        written.add(write_idx[i])
        assert torch.equal(pre_got[s].float(), x[i]), f"request {i} pre-conv rows"
    for r in range(2 * R + 1):  # every ring row the step does not write keeps its bits (the read rows too)
        if r not in written:
            assert torch.equal(ring_got[r], ring[r]), f"ring row {r} changed"
    for s in range(R + 1):
        if s not in slots:
            assert torch.equal(pre_got[s].float(), pre_pool[s])


def packed_layer_inputs(g0, lens, C, Hv):
    total = sum(lens)
    x = G.bf16_round(torch.randn(total, C, generator=g0))
    a_in = G.bf16_round(torch.randn(total, Hv, generator=g0))
    b_in = G.bf16_round(torch.randn(total, Hv, generator=g0))
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    return x, a_in, b_in, cu


@pytest.mark.parametrize("geo", [(2, 4, 32, 16), (16, 16, 128, 128)])
def test_packed_prep_and_recurrent_with_pools(gpu, geo):
    """A packed ragged batch (cu_seqlens) through gdn_prep (conv_bias, window pool by win_idx, pre-conv pool
    by pre_idx, new windows into a pool) and gdr_recurrent (state pool by state_idx updated in place,
    intermediate states into a ring by inter_idx, cache_steps = 4, canvas readout num_clean = 2)."""
    Hk, Hv, Dk, Dv = geo
    g0 = torch.Generator().manual_seed(100 + Dk)
    lens = [5, 1, 9, 3]
    B, Tmax, N, nclean = len(lens), max(lens), 4, 2
    C, conv_w, conv_b, A_log, dt = layer_weights(g0, Hk, Hv, Dk, Dv)
    x, a_in, b_in, cu = packed_layer_inputs(g0, lens, C, Hv)
    win_idx, pre_idx, st_idx, int_idx = [2, 5, 0, 3], [1, 3, 0, 4], [4, 1, 5, 0], [2, 0, 3, 1]
    win_pool = G.bf16_round(torch.randn(6, 3, C, generator=g0))
    pool = torch.randn(6, Hv, Dv, Dk, generator=g0) * 0.1
    ring = torch.randn(4, N, Hv, Dv, Dk, generator=g0)

    cu_d = i32(cu)
    wout_d = torch.zeros(6, 3, C, dtype=torch.bfloat16, device=DEV)
    pre_d = torch.zeros(5, Tmax, C, dtype=torch.bfloat16, device=DEV)
    q, k, v, g, beta = kernels.gdn_prep(bf(x), bf(win_pool), bf(conv_w), bf(a_in), bf(b_in), A_log.to(DEV), dt.to(DEV),
                                        Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, window_out=wout_d, pre_out=pre_d,
                                        conv_bias=bf(conv_b), win_idx=i32(win_idx), pre_idx=i32(pre_idx),
                                        cu_seqlens=cu_d, max_rows=Tmax)
    pool_d, ring_d = pool.to(DEV).contiguous(), ring.to(DEV).contiguous()
    out, clean = kernels.gdr_recurrent(q, k, v, g, beta, pool_d, causal_mode=2, num_clean=nclean, state_out=pool_d,
                                       want_clean=True, cu_seqlens=cu_d, max_rows=Tmax, state_idx=i32(st_idx),
                                       inter=ring_d, inter_idx=i32(int_idx), cache_steps=N)
    torch.cuda.synchronize()
    pool_got, ring_got, wout, pre = pool_d.cpu(), ring_d.cpu(), wout_d.cpu().float(), pre_d.cpu().float()
    for b, L in enumerate(lens):
        r0, r1 = cu[b], cu[b + 1]
        rq, rk, rv, rg, rb, rwin = G.prep(x[None, r0:r1], win_pool[win_idx[b]][None], conv_w, a_in[None, r0:r1],
                                          b_in[None, r0:r1], A_log, dt, Hk, Hv, Dk, Dv, conv_bias=conv_b)
        for got, ref, name in ((q, rq, "q"), (k, rk, "k"), (v, rv, "v")):
            assert rel(got[r0:r1], ref[0]) < TOL_BF16, f"sequence {b} {name}"
        assert rel(g[r0:r1], rg[0]) < 1e-5 and rel(beta[r0:r1], rb[0]) < 1e-5, f"sequence {b} gates"
        assert torch.equal(wout[win_idx[b]], rwin[0]), f"sequence {b} new window"
        assert torch.equal(pre[pre_idx[b], :L], x[r0:r1]), f"sequence {b} pre-conv rows"
        s0 = pool[st_idx[b]][None]
        o_ref, c_ref, s_end = G.canvas(rq, rk, rv, rg, rb, s0, num_clean=nclean, causal_mode=2)
        _, _, states = G.recurrent(rq, rk, rv, rg, rb, s0, record_states=True)
        assert rel(out[r0:r1], o_ref[0]) < TOL_BF16, f"sequence {b} readout"
        assert rel(pool_got[st_idx[b]], s_end[0]) < TOL_F32, f"sequence {b} final state in the pool"
        assert rel(clean[b], c_ref[0]) < TOL_F32, f"sequence {b} clean state"
        for j in range(N):  # rows past a short sequence's end are not written
            want = states[j][0] if j < L else ring[int_idx[b], j]
            assert rel(ring_got[int_idx[b], j], want) < TOL_F32, f"sequence {b} ring entry {j}"
    for r in set(range(6)) - set(st_idx):
        assert torch.equal(pool_got[r], pool[r])
    for r in set(range(6)) - set(win_idx):
        assert torch.equal(wout[r], torch.zeros(3, C))


@pytest.mark.parametrize("lens,causal_mode", [([130, 64, 1, 200], 1), ([33, 7, 64, 1], 2)])
def test_packed_chunk_with_state_pool(gpu, lens, causal_mode):
    """gdr_chunk over a packed ragged prefill (chunks split at each sequence's own boundaries) and over
    packed canvas blocks (T <= 64, the fused single-chunk kernel), state pool updated in place."""
    Hk, Hv, Dk, Dv = 4, 8, 128, 64
    g0 = torch.Generator().manual_seed(sum(lens))
    B, Tmax, total = len(lens), max(lens), sum(lens)
    q = G.bf16_round(G.l2norm(torch.randn(total, Hk, Dk, generator=g0)))
    k = G.bf16_round(G.l2norm(torch.randn(total, Hk, Dk, generator=g0)))
    v = G.bf16_round(torch.randn(total, Hv, Dv, generator=g0))
    g = -F.softplus(torch.randn(total, Hv, generator=g0))
    beta = torch.sigmoid(torch.randn(total, Hv, generator=g0))
    pool = torch.randn(B + 2, Hv, Dv, Dk, generator=g0) * 0.1
    st_idx = list(range(B + 1, 1, -1))  # reversed rows, two rows unused
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    pool_d = pool.to(DEV).contiguous()
    nclean = 3
    out = kernels.gdr_chunk(bf(q), bf(k), bf(v), g.to(DEV).contiguous(), beta.to(DEV).contiguous(), pool_d,
                            causal_mode=causal_mode, num_clean=nclean if causal_mode == 2 else None,
                            state_out=pool_d, cu_seqlens=i32(cu), max_rows=Tmax, state_idx=i32(st_idx))
    torch.cuda.synchronize()
    pool_got = pool_d.cpu()
    for b, L in enumerate(lens):
        r0, r1 = cu[b], cu[b + 1]
        s0 = pool[st_idx[b]][None]
        args = (q[None, r0:r1], k[None, r0:r1], v[None, r0:r1], g[None, r0:r1], beta[None, r0:r1], s0)
        if causal_mode == 2:
            o_ref, _, s_ref = G.canvas(*args, num_clean=nclean, causal_mode=2)
        else:
            o_ref, s_ref, _ = G.recurrent(*args)
        assert rel(out[r0:r1], o_ref[0]) < TOL_BF16, f"sequence {b} readout"
        assert rel(pool_got[st_idx[b]], s_ref[0]) < TOL_F32, f"sequence {b} state"
    for r in set(range(B + 2)) - set(st_idx):
        assert torch.equal(pool_got[r], pool[r])


def test_window_rebuild_over_layer_pools(gpu):
    """The self-spec sampler's conv-window rebuild for every layer in one launch, in place on the window
    pool: wc[:, slot + 1] = last 3 rows of (wc[:, slot + 1] ++ preconv[:, slot, :n_acc + 1])
    (qwen3_5_diffusion.py:963-975), through trida_gdn_restore's pool form."""
    g0 = torch.Generator().manual_seed(5)
    L, R, blk, C = 3, 5, 7, 192
    slots, n_acc = [3, 0, 4], [0, 2, 6]
    n = len(slots)
    wc = G.bf16_round(torch.randn(L, R + 2, 3, C, generator=g0))
    pre = G.bf16_round(torch.randn(L, R + 1, blk, C, generator=g0))
    sl = torch.tensor(slots)
    seq = torch.cat([wc[:, sl + 1], pre[:, sl]], dim=2)                           # [L, n, 3 + blk, C]
    gidx = (torch.tensor(n_acc)[:, None] + 1 + torch.arange(3)[None, :])          # [n, 3]
    want = wc.clone()
    want[:, sl + 1] = seq.gather(2, gidx[None, :, :, None].expand(L, -1, -1, C))
    wc_d = bf(wc)
    pool = wc_d.view(L * (R + 2), 3, C)
    win_idx = i32([l * (R + 2) + s + 1 for l in range(L) for s in slots])
    pre_idx = i32([l * (R + 1) + s for l in range(L) for s in slots])
    kernels.gdn_restore(i32([a + 1 for a in n_acc]), snap_window=pool, window=pool,
                        preconv=bf(pre).view(L * (R + 1), blk, C), win_idx=win_idx, pre_idx=pre_idx, slots=L * n)
    torch.cuda.synchronize()
    assert torch.equal(wc_d.cpu().float(), want)


def test_out_of_range_indices_are_refused_before_launch(gpu):
    """Pool / ring indices and cu_seqlens that would address memory outside their buffers raise on the host
    (the wrappers read them back outside graph capture); nothing is launched, the pools stay untouched."""
    g0 = torch.Generator().manual_seed(11)
    Hk, Hv, Dk, Dv, T = 2, 4, 32, 64, 5
    C = 2 * Hk * Dk + Hv * Dv
    x = bf(torch.randn(2, T, C, generator=g0))
    ab = bf(torch.randn(2, T, Hv, generator=g0))
    conv_w = bf(torch.randn(C, 4, generator=g0) * 0.3)
    A_log = torch.zeros(Hv, device=DEV)
    dt = torch.zeros(Hv, device=DEV)
    pool = bf(torch.randn(3, 3, C, generator=g0))
    before = pool.clone()
    with pytest.raises(ValueError, match="win_idx"):
        kernels.gdn_prep(x, pool, conv_w, ab, ab, A_log, dt, Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, win_idx=i32([0, 3]))
    with pytest.raises(ValueError, match="win_idx"):
        kernels.gdn_prep(x, pool, conv_w, ab, ab, A_log, dt, Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv, win_idx=i32([-1, 1]))
    assert torch.equal(pool, before)
    q = bf(torch.randn(2, T, Hk, Dk, generator=g0))
    v = bf(torch.randn(2, T, Hv, Dv, generator=g0))
    gl = -torch.rand(2, T, Hv, generator=g0).to(DEV)
    beta = torch.rand(2, T, Hv, generator=g0).to(DEV)
    states = torch.randn(3, Hv, Dv, Dk, generator=g0).to(DEV)
    s_before = states.clone()
    with pytest.raises(ValueError, match="state_idx"):
        kernels.gdr_recurrent(q, q, v, gl, beta, states, state_idx=i32([1, 5]))
    with pytest.raises(ValueError, match="distinct"):  # written in place: two sequences on one pool row
        kernels.gdr_recurrent(q, q, v, gl, beta, states, state_out=states, state_idx=i32([2, 2]))
    ring = torch.zeros(2, 3, Hv, Dv, Dk, device=DEV)
    with pytest.raises(ValueError, match="inter_idx"):
        kernels.gdr_recurrent(q, q, v, gl, beta, states, state_idx=i32([0, 1]), inter=ring, inter_idx=i32([0, 2]))
    qp, vp = q.view(2 * T, Hk, Dk), v.view(2 * T, Hv, Dv)
    with pytest.raises(ValueError, match="cu_seqlens"):
        kernels.gdr_recurrent(qp, qp, vp, gl.view(2 * T, Hv), beta.view(2 * T, Hv), states[:2],
                              cu_seqlens=i32([0, 6, 2 * T + 1]), max_rows=T + 1)
    with pytest.raises(ValueError, match="cu_seqlens"):
        kernels.gdr_recurrent(qp, qp, vp, gl.view(2 * T, Hv), beta.view(2 * T, Hv), states[:2],
                              cu_seqlens=i32([0, 7, 6]), max_rows=T + 2)
    assert torch.equal(states, s_before) and torch.equal(ring, torch.zeros_like(ring))
    # in range, the same calls run
    out, _ = kernels.gdr_recurrent(q, q, v, gl, beta, states, state_idx=i32([2, 0]))
    assert torch.isfinite(out.float()).all()
