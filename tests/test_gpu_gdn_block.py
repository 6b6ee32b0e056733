"""GPU parity: the single-block MFMA readout of the gated delta rule (gdn_block.hip, reached through
trida_gdr_chunk for readout-only blocks with Dk = 128) against the CPU oracle's token-recurrent canvas
readout (oracle.gdn.canvas, pinned to transformers' fixtures). Tolerance as the other GDN forms: bf16 outputs
1e-2 normwise."""
import pytest
import torch

from oracle import gdn as G
from trida_stack_amd import kernels
from test_gpu_gdn import TOL_BF16, gdr_inputs, rel, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T,Hk,Hv,Dv", [
    (1, 33, 16, 16, 128),   # the 4B verify block at batch 1 (one wave per 32 columns)
    (8, 33, 16, 16, 128),   # batch 8: one workgroup per head (4 waves)
    (1, 1, 2, 2, 128),      # an AR row
    (2, 16, 4, 8, 128),     # one row tile, GQA
    (2, 17, 4, 8, 256),     # a ragged second tile, Dv 256
    (1, 48, 2, 2, 128),
    (3, 64, 2, 4, 128),     # the largest block
])
@pytest.mark.parametrize("mode,nc", [(1, None), (2, 0), (2, 1), (2, 9)])
def test_gdr_block_matches_oracle(gpu, B, T, Hk, Hv, Dv, mode, nc):
    shape = (B, T, Hk, Hv, 128, Dv)
    inp = gdr_inputs(7 * T + B + Dv + (nc or 0), *shape)
    n = T if nc is None else min(nc, T)
    o_ref, _, _ = G.canvas(*inp, num_clean=n, causal_mode=mode)
    q, k, v, g, beta, s0 = to_dev(*inp)
    o = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=mode, num_clean=n)
    assert rel(o, o_ref) < TOL_BF16, rel(o, o_ref)
    assert torch.equal(s0.cpu(), inp[5]), "the state is read only"


def test_gdr_block_strong_decay_and_large_state(gpu):
    """Log decays down to -30 per row and a state of norm ~10: every exponent taken is <= 0."""
    B, T, Hk, Hv, Dk, Dv = 2, 33, 4, 4, 128, 128
    q, k, v, g, beta, s0 = gdr_inputs(11, B, T, Hk, Hv, Dk, Dv, state_scale=3.0)
    g = -torch.rand(B, T, Hv, generator=torch.Generator().manual_seed(3)) * 30
    for mode, nc in ((1, T), (2, 1)):
        o_ref, _, _ = G.canvas(q, k, v, g, beta, s0, num_clean=nc, causal_mode=mode)
        o = kernels.gdr_chunk(*to_dev(q, k, v, g, beta, s0), causal_mode=mode, num_clean=nc)
        assert torch.isfinite(o.float()).all()
        assert rel(o, o_ref) < TOL_BF16


def test_gdr_block_agrees_with_recurrent_kernel_batch64(gpu):
    """The two GPU forms of the 4B canvas block at batch 64 (the large-grid path): verify and draft."""
    inp = gdr_inputs(5, 64, 33, 16, 16, 128, 128)
    q, k, v, g, beta, s0 = to_dev(*inp)
    for mode, nc in ((1, 33), (2, 1)):
        o1, _ = kernels.gdr_recurrent(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc)
        o2 = kernels.gdr_chunk(q, k, v, g, beta, s0, causal_mode=mode, num_clean=nc)
        assert rel(o2, o1) < TOL_BF16
