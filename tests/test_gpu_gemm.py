"""GPU parity: the weight-streaming bf16 GEMM (pre-shuffled weights; bf16, fp32-partial and SwiGLU
epilogues) and add_rmsnorm over partial planes, against fp32 torch references of the same ops."""
import pytest
import torch
import torch.nn.functional as F

from trida_stack_amd import kernels as TK

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def shuffle_ref(w, pair=False):
    """The layout from its definition: tile t, k-step s, lane 16 g + r -> W[row][32 s + 8 g .. + 8]."""
    N, K = w.shape
    if pair:  # tile t = 8 gate rows 8t.. then the 8 matching up rows
        g, u = w[: N // 2], w[N // 2:]
        w = torch.stack([g.view(N // 16, 8, K), u.view(N // 16, 8, K)], 1).reshape(N, K)
    return w.view(N // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)


def run(x, w, epi):
    """ws_gemm of x [M, K] against w [N, K]; returns the fp32 result [M, N] (or [M, N / 2] for SwiGLU)."""
    M, K = x.shape
    N = w.shape[0]
    wp = TK.ws_shuffle(w, pair_halves=epi == TK.WS_SILU)
    if epi == TK.WS_PARTS:
        kg = TK.ws_plan(N, K, epi)
        out = torch.full((kg * M * N,), float("nan"), dtype=torch.float32, device=DEV)
        TK.ws_gemm(x, wp, N, out, epilogue=epi)
        return out.view(kg, M, N).sum(0), out.view(kg, M, N)
    width = N // 2 if epi == TK.WS_SILU else N
    out = torch.empty(M, width, dtype=torch.bfloat16, device=DEV)
    TK.ws_gemm(x, wp, N, out, epilogue=epi)
    return out.float(), out


@pytest.mark.parametrize("pair", [False, True])
def test_shuffle_layout(gpu, pair):
    g = torch.Generator().manual_seed(1)
    w = torch.randn(64, 96, generator=g).to(torch.bfloat16)
    wp = TK.ws_shuffle(w.to(DEV), pair_halves=pair)
    assert torch.equal(wp.cpu(), shuffle_ref(w, pair))


@pytest.mark.parametrize("M,N,K", [
    (33, 8224, 2560),    # GDN in-projection
    (33, 10240, 2560),   # attention qkv
    (1, 8224, 2560),     # an AR row
    (48, 512, 2560),     # the largest M
    (7, 16, 32),         # minimum sizes
    (17, 48, 96),
])
def test_ws_store(gpu, M, N, K):
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    ref = x.float() @ w.float().t()
    y, _ = run(x.to(DEV), w.to(DEV), TK.WS_STORE)
    assert rel(y, ref) < 1e-2


@pytest.mark.parametrize("M,N,K", [
    (33, 2560, 9728),    # MLP down
    (33, 2560, 4096),    # attention out-projection
    (33, 2560, 2048),    # GDN out-projection
    (5, 64, 32 * 333),   # k-steps not a multiple of any wave slice: zero-padded tail steps
    (48, 32, 64),
])
def test_ws_parts(gpu, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    ref = x.float() @ w.float().t()
    y, planes = run(x.to(DEV), w.to(DEV), TK.WS_PARTS)
    assert torch.isfinite(planes).all()  # every plane element written
    assert rel(y, ref) < 2e-3  # fp32 partial sums: only the accumulation order differs


@pytest.mark.parametrize("M,I,K", [(33, 9728, 2560), (1, 9728, 2560), (9, 128, 64)])
def test_ws_silu(gpu, M, I, K):
    g = torch.Generator().manual_seed(M + I)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, generator=g) * 0.05).to(torch.bfloat16)
    gu = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    ref = F.silu(gu[:, :I]) * gu[:, I:]
    y, _ = run(x.to(DEV), w.to(DEV), TK.WS_SILU)
    assert y.shape == (M, I)
    assert rel(y, ref) < 2e-2


@pytest.mark.parametrize("epi,N,K", [(0, 8224, 2560), (1, 2560, 9728), (2, 19456, 2560)])
def test_ws_rows_independent_of_m(gpu, epi, N, K):
    """The plan depends on (N, K, epilogue) only: row i of the result is bitwise the same for any M."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(48, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    full, _ = run(x, w, epi)
    for M in (1, 7, 16, 17, 33):
        part, _ = run(x[:M].contiguous(), w, epi)
        assert torch.equal(part, full[:M]), f"M={M}"


def test_ws_strided_rows(gpu):
    """X rows and bf16 out rows with padded strides."""
    g = torch.Generator().manual_seed(3)
    xb = torch.randn(33, 2560 + 64, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(10240, 2560, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    ref = xb[:, :2560].float() @ w.float().t()
    wp = TK.ws_shuffle(w)
    y = torch.zeros(33, 10240 + 32, dtype=torch.bfloat16, device=DEV)
    TK.ws_gemm(xb[:, :2560], wp, 10240, y[:, :10240], epilogue=TK.WS_STORE)
    assert rel(y[:, :10240], ref) < 1e-2
    assert not y[:, 10240:].any()  # nothing written past N


def test_ws_rejects_bad_shapes(gpu):
    x = torch.zeros(49, 64, dtype=torch.bfloat16, device=DEV)
    wp = torch.zeros(32 * 64, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(49, 32, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        TK.ws_gemm(x, wp, 32, out)  # M > 48
    with pytest.raises(ValueError):
        TK.ws_plan(2560, 9728, TK.WS_STORE)  # K too long for a whole-K epilogue


@pytest.mark.parametrize("n_parts", [1, 4])
def test_add_rmsnorm_parts(gpu, n_parts):
    """Bitwise the add_rmsnorm of the bf16-rounded plane sum (summed in plane order)."""
    g = torch.Generator().manual_seed(n_parts)
    rows, dim = 33, 2560
    h = torch.randn(rows, dim, generator=g).to(torch.bfloat16).to(DEV)
    parts = (torch.randn(n_parts, rows, dim, generator=g) * 0.5).to(DEV)
    w = (torch.randn(dim, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    acc = parts[0].clone()
    for s in range(1, n_parts):
        acc += parts[s]
    r = acc.to(torch.bfloat16)
    h_ref, out_ref = h.clone(), torch.empty(rows, dim, dtype=torch.bfloat16, device=DEV)
    TK.add_rmsnorm(h_ref, r, w, out_ref)
    out = torch.empty_like(out_ref)
    TK.add_rmsnorm_parts(h, parts, n_parts, w, out)
    assert torch.equal(h, h_ref) and torch.equal(out, out_ref)
