"""GPU parity: canvas attention kernel vs the CPU oracle (tolerance 2e-2, normwise max-abs)."""
import pytest
import torch

from oracle import attention as A
from trida_stack_amd import kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 2e-2


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def inputs(seed, B, T, Hq, Hkv, D, L):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16)
    return q, kc, vc


CASES = [  # B, T, Hq, Hkv, D, L, prefixes
    (1, 32, 16, 4, 256, 8224, [8192]),          # config 3: verify / draft over 8192 + 32
    (1, 33, 16, 4, 256, 2400, [2100]),          # the 4B-shape canvas (132 query rows)
    (2, 5, 4, 2, 64, 300, [0, 213]),
    (3, 9, 8, 2, 128, 520, [1, 77, 500]),
    (1, 40, 8, 2, 128, 200, [100]),             # 160 query rows: two query tiles
    # ragged batches whose (sequence, KV head) pairs fill whole XCD rounds: scheduled longest-first
    (4, 7, 8, 2, 64, 400, [5, 390, 120, 390]),
    (8, 33, 16, 4, 256, 700, [600, 10, 333, 600, 0, 59, 512, 256]),
    # 20 sequences x 4 KV heads x 2 query tiles: one key split per tile
    (20, 33, 16, 4, 256, 300, [(37 * i) % 260 for i in range(20)]),
    # more query tiles than CUs: a last tile of 4 rows joins the tile before it as its extra rows (one key
    # split; two with 256 (sequence, KV head) pairs), a last tile of 44 rows stays a tile (two splits), as
    # does a single tile of 64 rows
    (40, 33, 16, 4, 256, 500, [(97 * i) % 460 for i in range(40)]),
    (48, 65, 8, 2, 64, 300, [(53 * i) % 236 for i in range(48)]),
    (128, 33, 8, 2, 64, 200, [(71 * i) % 167 for i in range(128)]),
    (64, 33, 16, 4, 128, 160, [(31 * i) % 127 for i in range(64)]),
    (48, 75, 8, 2, 64, 300, [(29 * i) % 226 for i in range(48)]),
    (136, 16, 8, 2, 64, 200, [(41 * i) % 185 for i in range(136)]),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_attn_canvas(gpu, case, mode):
    B, T, Hq, Hkv, D, L, prefix = case
    q, kc, vc = inputs(B + T + D + mode, B, T, Hq, Hkv, D, L)
    nc = T // 2
    ref = A.canvas_attention(q, kc, vc, prefix, mode, nc)
    out = kernels.attn_canvas(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor(prefix, dtype=torch.int32, device=DEV),
                              mask_mode=mode, n_clean=nc)
    assert rel(out, ref) < TOL


@pytest.mark.parametrize("splits", [1, 3, 64, 200])
def test_attn_split_counts(gpu, splits):
    B, T, Hq, Hkv, D, L, prefix = 1, 33, 16, 4, 256, 1100, [1000]
    q, kc, vc = inputs(7, B, T, Hq, Hkv, D, L)
    ref = A.canvas_attention(q, kc, vc, prefix, 0)
    out = kernels.attn_canvas(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor(prefix, dtype=torch.int32, device=DEV),
                              mask_mode=0, splits=splits)
    assert rel(out, ref) < TOL


@pytest.mark.parametrize("splits", [0, 1])
def test_attn_gate_and_crop(gpu, splits):
    """Output gate fused into the combine (or, with one key split, into the partial kernel's own output);
    a KV crop is only a prefix-length change."""
    B, T, Hq, Hkv, D, L = 1, 8, 8, 2, 128, 64
    q, kc, vc = inputs(3, B, T, Hq, Hkv, D, L)
    gate = torch.randn(B, T, Hq, 2 * D).to(torch.bfloat16)[..., D:]  # interleaved [q | gate] per head
    for prefix in (30, 21):  # second call: the cache was cropped back to 21 committed keys
        ref = A.canvas_attention(q, kc, vc, [prefix], 0, gate=gate)
        out = kernels.attn_canvas(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor([prefix], dtype=torch.int32, device=DEV),
                                  mask_mode=0, gate=gate.to(DEV), splits=splits)
        assert rel(out, ref) < TOL


def test_attn_one_split_equals_combine(gpu):
    """One key split: the partial kernel's direct (gated) output is bitwise what the combine writes from
    the same single split, row-major and in fragment order."""
    g = torch.Generator().manual_seed(11)
    B, T, Hq, Hkv, D, L = 1, 33, 16, 4, 256, 300
    q = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    kc = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16).to(DEV)
    gate = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    pl = torch.tensor([200], dtype=torch.int32, device=DEV)
    ref = A.canvas_attention(q.cpu(), kc.cpu(), vc.cpu(), [200], 0, gate=gate.cpu())
    one = kernels.attn_canvas(q, kc, vc, pl, mask_mode=0, gate=gate, splits=1)
    assert rel(one, ref) < TOL
    of = torch.zeros(kernels.ws_frag_numel(Hq * D), dtype=torch.bfloat16, device=DEV)
    kernels.attn_canvas(q, kc, vc, pl, mask_mode=0, gate=gate, splits=1, out=of, out_frag=True)
    from test_gpu_wsfused import _frag_mask
    mask = _frag_mask(B * T, Hq * D)
    assert torch.equal(kernels.ws_frag(one.view(B * T, -1)).view(torch.int16).cpu()[mask],
                       of.view(torch.int16).cpu()[mask])


def test_attn_clean_rows_equal_verify_rows(gpu):
    """Canvas clean rows (mode 2, rows < n_clean) equal the verify (causal) rows exactly."""
    B, T, Hq, Hkv, D, L = 1, 33, 16, 4, 256, 600
    q, kc, vc = [t.to(DEV) for t in inputs(4, B, T, Hq, Hkv, D, L)]
    pl = torch.tensor([500], dtype=torch.int32, device=DEV)
    o0 = kernels.attn_canvas(q, kc, vc, pl, mask_mode=0)
    o2 = kernels.attn_canvas(q, kc, vc, pl, mask_mode=2, n_clean=17)
    assert torch.equal(o0[:, :17], o2[:, :17])


@pytest.mark.parametrize("case,splits", [
    ((1, 33, 16, 4, 256, 2400, [2100]), 2),                     # the 4B-shape canvas, two splits forced
    ((1, 33, 16, 4, 256, 64, [0]), 2),                          # one key block: the second split is empty
    ((40, 33, 16, 4, 256, 500, [(97 * i) % 460 for i in range(40)]), 2),  # a batch: two splits of its plan
    ((3, 9, 8, 2, 128, 520, [1, 77, 500]), 2),
    ((4, 7, 8, 2, 64, 400, [5, 390, 120, 390]), 2),
])
@pytest.mark.parametrize("mode", [0, 2])
def test_attn_two_split_combine_equals_general(gpu, case, splits, mode):
    """The one-round-trip combine of two splits writes bitwise what the general combine writes (gated and
    not, row-major and in fragment order), and both match the oracle."""
    from trida_stack_amd import _lib
    B, T, Hq, Hkv, D, L, prefix = case
    q, kc, vc = [t.to(DEV) for t in inputs(B * 3 + T + D + mode, B, T, Hq, Hkv, D, L)]
    g = torch.Generator().manual_seed(B + D)
    gate = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    pl = torch.tensor(prefix, dtype=torch.int32, device=DEV)
    nc = T // 2
    lib = _lib.load()
    for gt in (None, gate):
        fast = kernels.attn_canvas(q, kc, vc, pl, mask_mode=mode, n_clean=nc, gate=gt, splits=splits)
        assert lib.trida_attn_set_combine_general(1) == 0
        try:
            general = kernels.attn_canvas(q, kc, vc, pl, mask_mode=mode, n_clean=nc, gate=gt, splits=splits)
        finally:
            lib.trida_attn_set_combine_general(0)
        assert torch.equal(fast.view(torch.int16), general.view(torch.int16))
        ref = A.canvas_attention(q.cpu(), kc.cpu(), vc.cpu(), prefix, mode, nc, gate=None if gt is None else gt.cpu())
        assert rel(fast, ref) < TOL
    if B * T <= 48:
        of = torch.zeros(kernels.ws_frag_numel(Hq * D), dtype=torch.bfloat16, device=DEV)
        kernels.attn_canvas(q, kc, vc, pl, mask_mode=mode, n_clean=nc, gate=gate, splits=splits, out=of,
                            out_frag=True)
        from test_gpu_wsfused import _frag_mask
        mask = _frag_mask(B * T, Hq * D)
        assert torch.equal(kernels.ws_frag(fast.view(B * T, -1)).view(torch.int16).cpu()[mask],
                           of.view(torch.int16).cpu()[mask])
