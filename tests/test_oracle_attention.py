"""Pins the attention oracle (CPU): mask semantics of the reference canvas mask and torch SDPA."""
import torch
import torch.nn.functional as F

from oracle import attention as A


def test_canvas_mask_matches_reference_formula():
    # inner = (c <= r) | (r >= n_clean), prefix all visible (inference/zoro-1/mlx/trida_mlx/model.py:461-470)
    T, n, P = 7, 4, 3
    m = A.canvas_mask(P, T, 2, n)
    for r in range(T):
        for c in range(P + T):
            want = c < P or (c - P) <= r or r >= n
            assert bool(m[r, c]) == want
    assert A.canvas_mask(P, T, 0).sum() == T * P + T * (T + 1) // 2
    assert A.canvas_mask(P, T, 1).all()
    assert torch.equal(A.canvas_mask(P, T, 2, T), A.canvas_mask(P, T, 0))  # all rows clean == causal
    assert torch.equal(A.canvas_mask(P, T, 2, 0), A.canvas_mask(P, T, 1))  # no clean rows == draft


def test_attention_matches_sdpa():
    g = torch.Generator().manual_seed(0)
    B, T, Hq, Hkv, D, L = 2, 5, 4, 2, 16, 20
    q = torch.randn(B, T, Hq, D, generator=g)
    kc = torch.randn(B, Hkv, L, D, generator=g)
    vc = torch.randn(B, Hkv, L, D, generator=g)
    prefix = [6, 11]
    for mode, nc in ((0, 0), (1, 0), (2, 2)):
        out = A.canvas_attention(q, kc, vc, prefix, mode, nc)
        for b in range(B):
            n = prefix[b] + T
            k = kc[b, :, :n].repeat_interleave(Hq // Hkv, 0)
            v = vc[b, :, :n].repeat_interleave(Hq // Hkv, 0)
            ref = F.scaled_dot_product_attention(q[b].transpose(0, 1), k, v,
                                                 attn_mask=A.canvas_mask(prefix[b], T, mode, nc))
            assert torch.allclose(out[b], ref.transpose(0, 1), atol=1e-5)


def test_crop_then_verify_equals_shorter_prefix():
    """A KV crop is a length change: attention over a cropped prefix equals a cache built that short."""
    g = torch.Generator().manual_seed(1)
    B, T, H, D, L = 1, 3, 2, 8, 16
    q = torch.randn(B, T, H, D, generator=g)
    kc = torch.randn(B, H, L, D, generator=g)
    vc = torch.randn(B, H, L, D, generator=g)
    # cache holds 5 committed keys then a rejected tail; the new block is written at position 5
    full = A.canvas_attention(q, kc, vc, [5], 0)
    short_k = torch.cat([kc[:, :, :5], kc[:, :, 5:8]], dim=2)
    short_v = torch.cat([vc[:, :, :5], vc[:, :, 5:8]], dim=2)
    assert torch.allclose(full, A.canvas_attention(q, short_k, short_v, [5], 0))
