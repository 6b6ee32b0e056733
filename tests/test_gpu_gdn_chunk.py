"""GPU parity: the chunked (WY / UT, MFMA) gated delta rule vs the CPU oracle.

The oracle's recurrent and chunked forms are pinned to transformers' torch fixtures and to each other
(tests/test_oracle_gdn.py). Tolerances (normwise, max-abs error / max-abs reference): bf16 outputs
1e-2, fp32 states 1e-3.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as G
from trida_stack_amd import kernels
from test_gpu_gdn import TOL_BF16, TOL_F32, gdr_inputs, rel, to_dev

pytestmark = pytest.mark.gpu


SHAPES = [  # (B, T, Hk, Hv, Dk, Dv)
    (1, 1, 2, 2, 32, 16),        # an AR step
    (2, 7, 2, 4, 32, 64),        # a small canvas block (fused kernel, 32-row chunk), GQA
    (1, 33, 16, 16, 128, 128),   # one verify block of the 4B-shape model (fused, 64-row chunk)
    (3, 64, 4, 4, 64, 32),       # exactly one chunk
    (1, 65, 2, 2, 128, 32),      # two chunks, the second of one row
    (2, 200, 2, 4, 64, 64),      # several chunks, a ragged last chunk
    (1, 300, 4, 4, 128, 128),
    (2, 200, 2, 4, 128, 64),     # the one-launch prefix kernel (Dk 128, T > 64): GQA, batch 2, ragged
    (1, 130, 2, 2, 128, 256),    # 16 value-column slices per head
]


@pytest.mark.parametrize("shape", SHAPES)
def test_gdr_chunk_causal(gpu, shape):
    B, T, Hk, Hv, Dk, Dv = shape
    inp = gdr_inputs(100 + sum(shape), *shape)
    o_ref, s_ref, _ = G.recurrent(*inp)
    q, k, v, g, beta, s0 = to_dev(*inp)
    s_out = torch.empty_like(s0)
    o = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=1, state_out=s_out)
    assert rel(o, o_ref) < TOL_BF16, rel(o, o_ref)
    assert rel(s_out, s_ref) < TOL_F32, rel(s_out, s_ref)
    assert torch.equal(s0.cpu(), inp[5]), "state_in must be left untouched"


def test_gdr_chunk_state_in_place_and_strong_decay(gpu):
    """state_out aliasing state_in; log decays down to -30 per row (in-chunk cumulative decay far below
    the fp32 range of e^G): every exponent the kernel takes is <= 0, so nothing overflows."""
    B, T, Hk, Hv, Dk, Dv = 1, 130, 2, 2, 64, 32
    q, k, v, g, beta, s0 = gdr_inputs(7, B, T, Hk, Hv, Dk, Dv)
    g = -torch.rand(B, T, Hv, generator=torch.Generator().manual_seed(3)) * 30
    o_ref, s_ref, _ = G.recurrent(q, k, v, g, beta, s0)
    qd, kd, vd, gd, bd, sd = to_dev(q, k, v, g, beta, s0)
    o = kernels.gdr_chunk(qd, kd, vd, gd, bd, sd, state_out=sd)
    assert torch.isfinite(o.float()).all() and torch.isfinite(sd).all()
    assert rel(o, o_ref) < TOL_BF16 and rel(sd, s_ref) < TOL_F32


@pytest.mark.parametrize("T", [129, 257])
def test_gdr_prefix_state_only_and_strong_decay(gpu, T):
    """The prefix kernel (Dk 128, T > 64) without a readout (state only), and with log decays down to
    -30 per row: every exponent it takes is <= 0."""
    B, Hk, Hv, Dk, Dv = 2, 2, 2, 128, 32
    q, k, v, g, beta, s0 = gdr_inputs(T, B, T, Hk, Hv, Dk, Dv)
    g = -torch.rand(B, T, Hv, generator=torch.Generator().manual_seed(T)) * 30
    o_ref, s_ref, _ = G.recurrent(q, k, v, g, beta, s0)
    qd, kd, vd, gd, bd, sd = to_dev(q, k, v, g, beta, s0)
    s_out = torch.full_like(sd, float("nan"))
    assert kernels.gdr_chunk(None, kd, vd, gd, bd, sd, state_out=s_out, want_out=False) is None
    assert rel(s_out, s_ref) < TOL_F32
    o = kernels.gdr_chunk(qd, kd, vd, gd, bd, sd, state_out=sd)  # in place
    assert torch.isfinite(o.float()).all() and torch.isfinite(sd).all()
    assert rel(o, o_ref) < TOL_BF16 and rel(sd, s_ref) < TOL_F32


@pytest.mark.parametrize("T,nc", [(7, 0), (7, 1), (7, 4), (7, 7), (33, 1), (33, 17), (64, 33), (20, 9)])
def test_gdr_chunk_canvas_block_end_readout(gpu, T, nc):
    shape = (2, T, 2, 4, 64, 32)
    inp = gdr_inputs(31 + T + nc, *shape)
    o_ref, _, se_ref = G.canvas(*inp, num_clean=nc, causal_mode=2)
    q, k, v, g, beta, s0 = to_dev(*inp)
    s_out = torch.empty_like(s0)
    o = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=2, num_clean=nc, state_out=s_out)
    assert rel(o, o_ref) < TOL_BF16
    assert rel(s_out, se_ref) < TOL_F32


def test_gdr_chunk_matches_recurrent_kernel_4b_block(gpu):
    """Both GPU forms of the 4B-shape canvas block at batch 8 agree (same readout contract)."""
    inp = gdr_inputs(5, 8, 33, 16, 16, 128, 128)
    q, k, v, g, beta, s0 = to_dev(*inp)
    for mode, nc in ((1, 33), (2, 1), (2, 12)):
        o1, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc)
        o2 = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc)
        assert rel(o2, o1) < TOL_BF16


@pytest.mark.parametrize("T", [33, 150])
def test_gdr_chunk_rollback_n_keep(gpu, T):
    """n_keep: the state after an accepted prefix of the block, from the block-entry state (the
    commit / rollback), per sequence, with slots stacked [layers x sequences] (seq_mod)."""
    L, B = 2, 3
    NB = L * B
    inp = gdr_inputs(40 + T, NB, T, 2, 4, 64, 32)
    q, k, v, g, beta, s0 = inp
    keep = [0, 5, T]
    n_keep = torch.tensor(keep, dtype=torch.int32)
    qd, kd, vd, gd, bd, sd = to_dev(*inp)
    s_out = torch.empty_like(sd)
    out = kernels.gdr_chunk(None, kd, vd, gd, bd, sd, state_out=s_out, n_keep=n_keep.to(sd.device), want_out=False)
    assert out is None
    for slot in range(NB):
        n = keep[slot % B]
        if n == 0:
            ref = s0[slot]
        else:
            _, ref, _ = G.recurrent(q[slot:slot + 1, :n], k[slot:slot + 1, :n], v[slot:slot + 1, :n],
                                    g[slot:slot + 1, :n], beta[slot:slot + 1, :n], s0[slot:slot + 1])
            ref = ref[0]
        assert rel(s_out[slot], ref) < TOL_F32, (slot, n)


def test_gdr_chunk_config2_prefix_block_rollback(gpu):
    """The config-2 workload at full size: batch 1, 16 heads, d_k = d_v = 128, a 4096-row prefix from
    a zero state (chunks of 64), then a 32-row verify block on top, snapshot before the block and
    rollback to an accepted length; against the oracle's chunked form on the host."""
    B, T, H, D = 1, 4096, 16, 128
    q, k, v, g, beta, _ = gdr_inputs(2024, B, T, H, H, D, D)
    s0 = torch.zeros(B, H, D, D)
    o_ref, s_ref = G.chunked(q, k, v, g, beta, s0)
    qd, kd, vd, gd, bd, sd = to_dev(q, k, v, g, beta, s0)
    o = kernels.gdr_chunk(qd, kd, vd, gd, bd, sd, state_out=sd)
    assert rel(o, o_ref) < TOL_BF16, rel(o, o_ref)
    assert rel(sd, s_ref) < TOL_F32, rel(sd, s_ref)
    # the 32-row block on top of the prefix state, canvas readout, then rollback to a = 19
    qb, kb, vb, gb, bb, _ = gdr_inputs(7, B, 32, H, H, D, D)
    ob_ref, _, _ = G.canvas(qb, kb, vb, gb, bb, s_ref, num_clean=17, causal_mode=2)
    blk = to_dev(qb, kb, vb, gb, bb, s_ref)
    snap = torch.empty_like(sd)
    kernels.gdn_snapshot(sd, snap)
    ob = kernels.gdr_chunk(*blk[:5], sd, causal_mode=2, num_clean=17)
    assert rel(ob, ob_ref) < TOL_BF16
    assert torch.equal(snap, sd), "the draft / verify pass must not write the state"
    a = 19
    kernels.gdr_chunk(None, *blk[1:5], snap, state_out=sd, want_out=False,
                      n_keep=torch.tensor([a], dtype=torch.int32, device=sd.device))
    _, sa_ref, _ = G.recurrent(qb[:, :a], kb[:, :a], vb[:, :a], gb[:, :a], bb[:, :a], s_ref)
    assert rel(sd, sa_ref) < TOL_F32


def test_gdr_chunk_rejects_bad_args(gpu):
    q, k, v, g, beta, s0 = to_dev(*gdr_inputs(1, 1, 70, 2, 2, 64, 32))
    with pytest.raises(ValueError, match="causal_mode 2"):
        kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=2, num_clean=3)
    q2, k2, v2, g2, b2, s2 = to_dev(*gdr_inputs(1, 1, 8, 2, 2, 256, 32))
    with pytest.raises(ValueError, match="Dk"):
        kernels.gdr_chunk(q2, k2, v2, g2, b2, s2)


def _recurrent_f64(q, k, v, g, beta, s0, causal_mode, num_clean):
    """S = e^g S; S += beta (v - S k) k^T; o = S q in fp64 on the device (block-end rows read the final S)."""
    q, k, v, S = q.double(), k.double(), v.double(), s0.double().clone()
    outs = []
    for t in range(v.shape[1]):
        S = S * g[:, t].double().exp()[:, :, None, None]
        kt = k[:, t][:, :, None, :]
        pred = (S * kt).sum(-1)
        S = S + beta[:, t].double()[:, :, None, None] * (v[:, t] - pred)[:, :, :, None] * kt
        outs.append((S * q[:, t][:, :, None, :]).sum(-1))
    o = torch.stack(outs, 1)
    if causal_mode == 2:
        for t in range(num_clean, v.shape[1]):
            o[:, t] = (S * q[:, t][:, :, None, :]).sum(-1)
    return o * q.shape[-1] ** -0.5


@pytest.mark.parametrize("mode,nc", [(1, 33), (2, 12)])
def test_gdr_block_batch64_correctly_rounded(gpu, mode, nc):
    """The canvas-block readout at the batch-64 verify shape (64 x 33 rows, 16 heads of 128 x 128): against an
    fp64 recurrence, >= 99% of the bf16 outputs are its correctly rounded value (the kernel's internal
    error stays below half a bf16 ulp almost everywhere) and the normwise error is that of the rounding."""
    q, k, v, g, beta, s0 = to_dev(*gdr_inputs(11, 64, 33, 16, 16, 128, 128))
    o = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc).double()
    r = _recurrent_f64(q, k, v, g, beta, s0, mode, nc)
    r16 = r.to(torch.bfloat16).double()
    assert float((o != r16).double().mean()) < 1e-2
    assert float((o - r).abs().mean()) < 1.05 * float((r16 - r).abs().mean())
    assert rel(o, r) < 5e-3


@pytest.mark.parametrize("T,nc", [(1, 1), (5, 2), (16, 16), (17, 3), (40, 40), (48, 20), (49, 49), (64, 31)])
def test_gdr_block_row_tiles(gpu, T, nc):
    """The canvas-block readout at each row-tile count (16, 32, 48 and 64 padded rows) and its edges,
    GQA (2 key heads for 4 value heads), two 128-column value groups per head, 3 sequences; causal rows
    for T == nc, else rows >= nc read the block-end state."""
    shape = (3, T, 2, 4, 128, 256)
    inp = gdr_inputs(500 + T, *shape)
    mode = 1 if nc == T else 2
    o_ref, _, _ = G.canvas(*inp, num_clean=nc, causal_mode=mode)
    q, k, v, g, beta, s0 = to_dev(*inp)
    o = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc)
    assert rel(o, o_ref) < TOL_BF16, rel(o, o_ref)
    assert torch.equal(s0.cpu(), inp[5]), "state_in must be left untouched"
