"""The weight-streaming GEMM's launch plan through the C ABI (host code only, no GPU): partial-plane counts
for the 4B-shape projections and the shapes it rejects."""
import pytest

from trida_stack_amd import kernels as TK


@pytest.mark.parametrize("N,K,epi,kg", [
    (19456, 2560, TK.WS_SILU, 1),     # MLP gate/up with the SwiGLU epilogue
    (8224, 2560, TK.WS_STORE, 1),     # GDN in-projection
    (10240, 2560, TK.WS_STORE, 1),    # attention qkv
    (16, 32, TK.WS_STORE, 1),
])
def test_whole_k_plans(N, K, epi, kg):
    assert TK.ws_plan(N, K, epi) == kg


@pytest.mark.parametrize("N,K", [(2560, 9728), (2560, 4096), (2560, 2048), (64, 32 * 333)])
def test_partial_plans_cover_k(N, K):
    kg = TK.ws_plan(N, K, TK.WS_PARTS)
    assert 1 <= kg <= 64
    # every plan's k-groups hold at most 80 k-steps (the largest whole-K slice) and cover K
    assert kg * 80 >= K // 32


def test_partial_plans_are_deterministic():
    assert [TK.ws_plan(2560, 9728, TK.WS_PARTS) for _ in range(3)] == [TK.ws_plan(2560, 9728, TK.WS_PARTS)] * 3


@pytest.mark.parametrize("N,K,epi", [
    (2560, 9728, TK.WS_STORE),   # K past one workgroup: only the partial-plane epilogue takes it
    (2560, 9728, TK.WS_SILU),
    (24, 64, TK.WS_STORE),       # N % 16
    (32, 48, TK.WS_PARTS),       # K % 32
    (32, 64, 7),                 # unknown epilogue
])
def test_rejected_plans(N, K, epi):
    with pytest.raises(ValueError):
        TK.ws_plan(N, K, epi)
