"""The fused unmasking of a denoise pass (trida_unmask_top) against the selection it replaces: a stable
descending sort of the masked slots' confidences, the first `count` slots taking their shifted
predictions."""
import pytest
import torch

from trida_stack_amd import kernels

DEV = torch.device("cuda:0")
pytestmark = pytest.mark.gpu


def reference(am, conf, masked, canvas, count):
    """torch on the CPU: where + stable sort + gather + scatter."""
    blk = masked.shape[1]
    score = torch.where(masked, conf[:, :blk], torch.full_like(conf[:, :blk], float("-inf")))
    pos = torch.sort(score, dim=1, descending=True, stable=True).indices[:, :count]
    canvas.scatter_(1, pos + 1, am[:, :blk].gather(1, pos))
    masked.scatter_(1, pos, False)


@pytest.mark.parametrize("B,blk,counts", [(1, 32, [8, 8, 8, 8]), (3, 32, [9, 8, 8, 7]), (2, 200, [0, 50, 1, 149]),
                                          (4, 5, [5])])
def test_unmask_top_matches_stable_sort(gpu, B, blk, counts):
    g = torch.Generator().manual_seed(B * 1000 + blk)
    canvas = torch.randint(0, 1000, (B, blk + 1), generator=g)
    masked = torch.ones(B, blk, dtype=torch.bool)
    d_canvas, d_masked = canvas.to(DEV), masked.to(DEV)
    for p, count in enumerate(counts):
        am = torch.randint(0, 50000, (B, blk + 1), generator=g)
        # few distinct values: many ties, which must resolve to the lower slot
        conf = torch.randint(0, 6, (B, blk + 1), generator=g).float() / 5
        reference(am, conf, masked, canvas, count)
        kernels.unmask_top(am.to(DEV), conf.to(DEV), d_masked, d_canvas, count)
        assert torch.equal(d_masked.cpu(), masked), p
        assert torch.equal(d_canvas.cpu(), canvas), p
    assert (masked.sum(1) == blk - sum(counts)).all()
