"""GPU parity: sampled acceptance (truncation statistics, truncated distributions, rejection sampling)
against the CPU oracle (oracle/accept.py). Decisions must match outside the oracle's flagged near-ties
(|u - ratio|, the nucleus boundary or an inverse-CDF step within 1e-6); ratios agree to 1e-5 relative,
the kept-set normaliser to 1e-6 relative."""
import numpy as np
import pytest
import torch

from oracle import accept as A
from trida_stack_amd import kernels as TK

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def y_of(logits, T, ban):
    y = np.asarray(logits, np.float32).copy()
    if ban >= 0:
        y[..., ban] = -np.inf
    if T != 1.0:
        y = (y / np.float32(T)).astype(np.float32)
    return y


def check_stats(logits, T, k, p, ban=-1, radix_only=False, expect_one_pass=None, max_passes=None):
    """GPU stats vs the oracle's kept set; returns the per-row pass counts."""
    x = torch.from_numpy(logits).to(DEV)
    m, thr, zk, st, passes = TK.truncate_stats(x, temperature=T, top_k=k, top_p=p, ban_id=ban,
                                              radix_only=radix_only, want_passes=True)
    m, thr, zk, st, passes = (t.cpu().numpy() for t in (m, thr, zk, st, passes))
    assert (st == 0).all()
    P, info = A.truncated_probs(logits, T, k, p, ban, return_info=True)
    y = y_of(logits, T, ban).astype(np.float64)
    B, R, V = logits.shape
    for b in range(B):
        for r in range(R):
            row = y[b, r]
            assert m[b, r] == np.float32(row.max())
            if info.boundary_gap[b, r] < 1e-6:
                continue  # a near-tie of the nucleus boundary: either side is correct
            fin = np.isfinite(row)
            kept_ref = info.kept[b, r] & fin
            kept_gpu = fin & (row >= thr[b, r])
            assert (kept_ref == kept_gpu).all(), (b, r, int(kept_ref.sum()), int(kept_gpu.sum()))
            zref = np.exp(row[kept_ref] - row.max()).sum()
            assert abs(zk[b, r] / zref - 1) < 1e-6, (b, r, zk[b, r], zref)
    # passes counts streamed quarter-rows: 4 = one pass over the row
    if expect_one_pass is not None:
        assert (passes == 4).mean() >= expect_one_pass, passes
    if max_passes is not None:
        assert passes.max() <= 4 * max_passes, passes
    return passes


@pytest.mark.parametrize("T,k,p", [(0.7, 0, 0.95), (1.0, 20, 0.95), (1.0, 50, 0.95), (0.7, 20, 0.8),
                                   (1.3, 5, 1.0), (0.7, 0, 1.0), (0.9, 4096, 0.9), (0.7, 0, 0.5)])
def test_truncate_stats_random(gpu, T, k, p):
    rng = np.random.default_rng(hash((T, k, p)) % 2**32)
    logits = (rng.normal(size=(3, 5, 5000)) * 3).astype(np.float32)
    check_stats(logits, T, k, p, expect_one_pass=0.9 if k <= 50 else None, max_passes=2)
    check_stats(logits, T, k, p, radix_only=True)


def test_truncate_stats_large_vocab(gpu):
    """A config-5 row width (V = 248320): the histogram pass resolves every typical row in at most two
    streaming passes (one when the sample-placed window holds the boundary)."""
    rng = np.random.default_rng(5)
    logits = (rng.normal(size=(2, 3, 248320)) * 2).astype(np.float32)
    check_stats(logits, 0.7, 0, 0.95, max_passes=2)
    check_stats(logits, 1.0, 20, 0.95, expect_one_pass=1.0)


def test_truncate_stats_fallbacks(gpu):
    """Rows the window path cannot resolve: a dominant token missed by the sample, massive ties, huge
    logits, banned ids and -inf entries, fewer finite entries than top_k, a vocabulary that is not a
    multiple of 4 (scalar loads)."""
    V = 3001
    rng = np.random.default_rng(9)
    rows = []
    r = rng.normal(size=V).astype(np.float32)
    r[1234] = 30.0  # one token holds nearly all the mass
    rows.append(r)
    rows.append(np.zeros(V, np.float32))  # every value tied
    r = (rng.normal(size=V) * 400).astype(np.float32)  # |y| in the thousands
    rows.append(r)
    r = rng.normal(size=V).astype(np.float32)
    r[::3] = -np.inf
    rows.append(r)
    r = np.full(V, -np.inf, np.float32)
    r[:7] = rng.normal(size=7)
    rows.append(r)
    r = np.round(rng.normal(size=V) * 2).astype(np.float32)  # few distinct values, many ties
    rows.append(r)
    logits = np.stack(rows)[None]
    for T, k, p in [(0.7, 0, 0.95), (1.0, 20, 0.95), (1.0, 50, 1.0), (0.5, 0, 0.3), (1.0, 2000, 0.99)]:
        check_stats(logits, T, k, p, ban=17)
        check_stats(logits, T, k, p, ban=17, radix_only=True)


def test_truncate_status_rows(gpu):
    x = torch.zeros((1, 3, 64), device=DEV)
    x[0, 0, 5] = float("nan")
    x[0, 1, :] = float("-inf")
    x[0, 2, 9] = float("inf")
    st = TK.truncate_stats(x, temperature=0.7, top_p=0.9)[3].cpu().tolist()
    assert st == [[1, 2, 1]]


def test_truncated_probs(gpu):
    rng = np.random.default_rng(2)
    logits = (rng.normal(size=(2, 4, 3000)) * 3).astype(np.float32)
    x = torch.from_numpy(logits).to(DEV)
    for T, k, p in [(0.7, 0, 0.95), (1.0, 20, 0.9), (1.2, 0, 1.0)]:
        stats = TK.truncate_stats(x, temperature=T, top_k=k, top_p=p, ban_id=3)
        P = TK.truncated_probs(x, stats, temperature=T, ban_id=3).cpu().numpy()
        ref = A.truncated_probs(logits, T, k, p, 3)
        assert np.abs(P - ref).max() < 2e-6
        assert np.allclose(P.sum(-1), 1, atol=1e-5)
        assert (P[..., 3] == 0).all()


@pytest.mark.parametrize("V", [3000, 3001])
def test_truncated_probs_rows_equals_gather_then_scatter(gpu, V):
    """Row-mapped P rows (vector path V % 4 == 0, scalar otherwise) == truncated_probs of the gathered
    rows, written at the mapped output rows, bit for bit; other rows and out-of-range indices untouched."""
    rng = np.random.default_rng(3)
    B, R, Ro, T = 3, 5, 7, 0.8
    x = torch.from_numpy((rng.normal(size=(B, R, V)) * 3).astype(np.float32)).to(DEV)
    stats = TK.truncate_stats(x, temperature=T, top_k=0, top_p=0.9, ban_id=2)[:3]
    full = TK.truncated_probs(x, stats, temperature=T, ban_id=2)
    in_rows = torch.tensor([[4, 0], [1, 1], [2, R]], dtype=torch.int64, device=DEV)  # (2, 1) out of range
    out_rows = torch.tensor([[6, 2], [0, 5], [3, 4]], dtype=torch.int64, device=DEV)
    out = torch.full((B, Ro, V), -1.0, device=DEV)
    TK.truncated_probs_rows(x, stats, in_rows, out_rows, out, temperature=T, ban_id=2)
    ref = torch.full_like(out, -1.0)
    for b in range(B):
        for j in range(2):
            i, o = int(in_rows[b, j]), int(out_rows[b, j])
            if i < R:
                ref[b, o] = full[b, i]
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 4096), (torch.bfloat16, 4099), (torch.float32, 4096),
                                     (torch.float32, 4099)])
def test_gather_rows_widens_exactly(gpu, dtype, V):
    g = torch.Generator(device=DEV).manual_seed(4)
    B, R, Kr = 2, 6, 4
    src = torch.randn(B, R, V, generator=g, device=DEV).to(dtype)
    rows = torch.tensor([[5, 0, 3, 3], [1, 6, 2, -1]], dtype=torch.int64, device=DEV)  # 6 and -1 skip
    out = torch.full((B, Kr, V), 7.0, device=DEV)
    TK.gather_rows(src, rows, out=out)
    ref = torch.full_like(out, 7.0)
    for b in range(B):
        for k in range(Kr):
            i = int(rows[b, k])
            if 0 <= i < R:
                ref[b, k] = src[b, i].float()
    assert torch.equal(out, ref)


def make_case(seed, B, K, V, T, k, p, accept_bias=2.0):
    """Verify logits and draft distributions q that overlap P (so drafts are often accepted)."""
    rng = np.random.default_rng(seed)
    base = (rng.normal(size=(B, K + 1, V)) * 3).astype(np.float32)
    pl = base
    ql = (base[:, :K] + rng.normal(size=(B, K, V)).astype(np.float32) / accept_bias).astype(np.float32)
    q = A.truncated_probs(ql, T, k, p).astype(np.float32)
    drafts = np.zeros((B, K), np.int64)
    for b in range(B):
        for i in range(K):
            qq = q[b, i].astype(np.float64)
            drafts[b, i] = rng.choice(V, p=qq / qq.sum())
    ua = rng.random((B, K)).astype(np.float32)
    us = rng.random(B).astype(np.float32)
    ctx = rng.integers(100, 5000, size=B)
    return pl, q, drafts, ua, us, ctx


def run_gpu(pl, q, drafts, ua, us, ctx, T, k, p, ban=-1, n_live=None):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    out = TK.sample_accept(t(pl), t(q), t(drafts), t(ua), t(us), temperature=T, top_k=k, top_p=p, ban_id=ban,
                           ctx_len=t(ctx.astype(np.int64)), n_live=None if n_live is None else t(n_live),
                           want_ratio=True)
    return [None if o is None else o.cpu().numpy() for o in out]


@pytest.mark.parametrize("T,k,p", [(0.7, 0, 0.95), (1.0, 20, 0.95), (1.0, 0, 1.0), (0.8, 50, 0.9)])
def test_sample_accept_vs_oracle(gpu, T, k, p):
    B, K, V = 12, 7, 4000
    pl, q, drafts, ua, us, ctx = make_case(11, B, K, V, T, k, p)
    n_acc, tok, crop, ratio, st = run_gpu(pl, q, drafts, ua, us, ctx, T, k, p)
    ref = A.rejection_accept(pl, q, drafts, ua, us, temperature=T, top_k=k, top_p=p, ctx_len=ctx)
    assert (st == 0).all()
    ok = ~ref["tie"]
    assert ok.sum() >= B - 2
    assert (n_acc[ok] == ref["n_acc"][ok]).all()
    assert (tok[ok] == ref["token"][ok]).all()
    assert (crop[ok] == ref["crop"][ok]).all()
    # ratios of the rows the decision used (up to the first rejection); the rows after it are never
    # evaluated and read 0
    used = np.arange(K)[None, :] <= n_acc[:, None]
    nz = used & (ref["ratio"] > 0)
    assert np.allclose(ratio[nz], ref["ratio"][nz], rtol=1e-5)
    assert (ratio[used & ~nz] == 0).all() and (ratio[~used] == 0).all()
    # the cases cover early rejections and full acceptance
    assert len(set(n_acc.tolist())) >= 3


def test_sample_accept_edges(gpu):
    """n_live limits, a banned MASK id, K = 0 (the bonus only), q = 0 on a draft, all accepted."""
    B, K, V = 6, 5, 1000
    T, k, p = 0.9, 0, 0.9
    pl, q, drafts, ua, us, ctx = make_case(4, B, K, V, T, k, p, accept_bias=20.0)
    q[0, 0, drafts[0, 0]] = 0.0  # ratio 0 -> reject at 0
    ua[1] = 0.0  # accept everything the ratio allows
    live = np.array([5, 5, 2, 0, 5, 3], np.int32)
    ban = 999
    n_acc, tok, crop, ratio, st = run_gpu(pl, q, drafts, ua, us, ctx, T, k, p, ban=ban, n_live=live)
    ref = A.rejection_accept(pl, q, drafts, ua, us, temperature=T, top_k=k, top_p=p, mask_id=ban, ctx_len=ctx)
    ref_n = ref["n_acc"].copy()
    for b in range(B):
        assert n_acc[b] <= live[b]
    assert n_acc[0] == 0
    assert (tok != ban).all()
    # sequences whose live limit does not bind follow the oracle exactly
    free = (ref_n <= live) & ~ref["tie"]
    assert (n_acc[free] == ref_n[free]).all() and (tok[free] == ref["token"][free]).all()
    # K = 0: the token is the bonus drawn from P_0
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    out = TK.sample_accept(t(pl[:, :1]), None, t(np.zeros((B, 0), np.int64)), None, t(us), temperature=T,
                           top_p=p)
    P0 = A.truncated_probs(pl[:, :1], T, 0, p)[:, 0]
    for b in range(B):
        tk, gap = A.sample_inverse_cdf(P0[b], float(us[b]))
        if gap > 1e-6:
            assert out[1][b].item() == tk and out[0][b].item() == 0


def test_sample_accept_config5_shape(gpu):
    """Batch 64, 33 verify rows, V = 248320 (q as full-vocabulary fp32 probabilities): the oracle checks
    eight of the sequences (the sequences are independent), the rest through invariants."""
    B, K, V = 64, 32, 248320
    T, k, p = 0.7, 0, 0.95
    g = torch.Generator(device="cpu").manual_seed(7)
    pl = (torch.randn(B, K + 1, V, generator=g) * 2)
    ql = pl[:, :K] + torch.randn(B, K, V, generator=g) * 0.3
    pg, qlg = pl.to(DEV), ql.to(DEV)
    qst = TK.truncate_stats(qlg, temperature=T, top_p=p)
    q = TK.truncated_probs(qlg, qst, temperature=T)
    del qlg
    drafts = torch.multinomial(q.reshape(-1, V), 1).reshape(B, K)
    ua = torch.rand(B, K, generator=g).to(DEV)
    us = torch.rand(B, generator=g).to(DEV)
    n_acc, tok, crop, ratio, st = TK.sample_accept(pg, q, drafts, ua, us, temperature=T, top_p=p, want_ratio=True)
    n_acc, tok = n_acc.cpu().numpy(), tok.cpu().numpy()
    assert (st.cpu().numpy() == 0).all()
    assert ((0 <= n_acc) & (n_acc <= K)).all() and ((0 <= tok) & (tok < V)).all()
    sel = list(range(0, B, 8))
    ref = A.rejection_accept(pl[sel].numpy(), q[sel].cpu().numpy(), drafts[sel].cpu().numpy(),
                             ua[sel].cpu().numpy(), us[sel].cpu().numpy(), temperature=T, top_p=p)
    ok = ~ref["tie"]
    assert (n_acc[sel][ok] == ref["n_acc"][ok]).all()
    assert (tok[sel][ok] == ref["token"][ok]).all()
