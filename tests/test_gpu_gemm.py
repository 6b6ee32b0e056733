"""GPU parity: the skinny bf16 GEMM vs an fp32 torch reference (the decode-step projection shapes)."""
import pytest
import torch

from trida_stack_amd import kernels as TK

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("M,N,K,splits", [
    (33, 19456, 2560, 0),   # SwiGLU gate/up
    (33, 2560, 9728, 0),    # down (split K)
    (33, 8224, 2560, 0),    # GDN in-projection
    (33, 2560, 2048, 0),    # GDN out-projection
    (1, 2560, 4096, 0),     # an AR row
    (64, 1040, 2560, 3),
    (17, 16, 32, 0),        # minimum sizes
    (50, 48, 96, 2),
])
def test_skinny_gemm(gpu, M, N, K, splits):
    g = torch.Generator().manual_seed(M * 7 + N)
    x = (torch.randn(M, K, generator=g)).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    ref = x.float() @ w.float().t()
    y = TK.linear(x.to(DEV), w.to(DEV), splits=splits)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert rel(y, ref) < 1e-2


def test_skinny_gemm_strided_out_and_lm_head(gpu):
    """Rows of X and Y with padded strides; an LM-head sized N (248320)."""
    g = torch.Generator().manual_seed(3)
    xb = torch.randn(33, 2560 + 64, generator=g).to(torch.bfloat16)
    w = (torch.randn(248320, 2560, generator=g) * 0.02).to(torch.bfloat16)
    ref = xb[:, :2560].float() @ w.float().t()
    x = xb.to(DEV)[:, :2560]
    y = torch.empty(33, 248320 + 16, dtype=torch.bfloat16, device=DEV)[:, :248320]
    TK.linear(x, w.to(DEV), out=y)
    assert rel(y, ref) < 1e-2
