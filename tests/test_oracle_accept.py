"""Pins the acceptance oracle (CPU): brute force, hand-computed cases and the reference's own
truncation spec (inference/zoro-1/mlx/tests/test_tiny.py:232-250)."""
import numpy as np
import pytest
import torch

from oracle import accept as A


def brute_argmax(row):
    best, bi = None, None
    for i, x in enumerate(row):
        if bi is None:
            best, bi = x, i
            continue
        if np.isnan(best):
            continue
        if np.isnan(x) or x > best:
            best, bi = x, i
    return bi


def test_argmax_first_ties_nan_inf():
    rows = np.array([
        [1.0, 3.0, 3.0, 2.0],
        [-np.inf, -np.inf, -np.inf, -np.inf],
        [0.0, np.nan, 5.0, np.nan],
        [np.inf, 1.0, np.nan, np.inf],
        [-0.0, 0.0, -1.0, 0.0],
    ], dtype=np.float32)
    got = A.argmax_first(rows)
    assert got.tolist() == [brute_argmax(r) for r in rows] == [1, 0, 1, 2, 0]
    # torch's CPU argmax agrees on the same rows
    assert got.tolist() == torch.from_numpy(rows).argmax(-1).tolist()


def decode_loop_greedy(vals, specs, live):
    """selfspec_generate's greedy verify (decode.py:326-329) as a loop."""
    acc = 0
    while acc < min(len(specs), live) and vals[acc] == specs[acc]:
        acc += 1
    return acc


@pytest.mark.parametrize("seed", range(6))
def test_greedy_accept_vs_loop(seed):
    rng = np.random.default_rng(seed)
    B, K, V = 5, 7, 11
    logits = rng.integers(-3, 4, size=(B, K + 1, V)).astype(np.float32)  # many ties on purpose
    am = np.array([[brute_argmax(r) for r in seq] for seq in logits])
    drafts = rng.integers(0, V, size=(B, K))
    for b in range(B):  # plant a matching prefix of random length
        n = rng.integers(0, K + 1)
        drafts[b, :n] = am[b, :n]
    live = rng.integers(0, K + 1, size=B).astype(np.int32)
    ctx = rng.integers(0, 100, size=B)
    g_am, n_acc, bonus, crop = A.greedy_accept(logits, drafts, live, ctx)
    assert (g_am == am).all()
    for b in range(B):
        acc = decode_loop_greedy(am[b].tolist(), drafts[b].tolist(), int(live[b]))
        assert n_acc[b] == acc
        assert bonus[b] == am[b, acc]
        assert crop[b] == ctx[b] + 1 + acc


def test_greedy_accept_hand_cases():
    V = 5
    eye = np.eye(V, dtype=np.float32)
    logits = np.stack([eye[[1, 2, 3, 4]]])  # rows predict 1, 2, 3, then bonus 4
    am, n, bonus, crop = A.greedy_accept(logits, np.array([[1, 2, 3]]), ctx_len=np.array([10]))
    assert (n.tolist(), bonus.tolist(), crop.tolist()) == ([3], [4], [14])
    am, n, bonus, crop = A.greedy_accept(logits, np.array([[0, 2, 3]]))
    assert (n.tolist(), bonus.tolist(), crop.tolist()) == ([0], [1], [1])
    am, n, bonus, crop = A.greedy_accept(logits, np.array([[1, 2, 0]]))
    assert (n.tolist(), bonus.tolist()) == ([2], [3])
    am, n, bonus, crop = A.greedy_accept(logits, np.array([[1, 2, 3]]), n_live=np.array([1]))
    assert (n.tolist(), bonus.tolist()) == ([1], [2])
    am, n, bonus, crop = A.greedy_accept(logits[:, :1], np.zeros((1, 0), np.int64))
    assert (n.tolist(), bonus.tolist()) == ([0], [1])


def test_greedy_workload_prefix():
    from trida_stack_amd import workloads

    w = workloads.greedy_accept_inputs(seed=3, batch=4, block=8, vocab=1000, ctx=50)
    _, n_acc, bonus, crop = A.greedy_accept(w["logits"].numpy(), w["drafts"].numpy(), ctx_len=w["ctx_len"].numpy())
    assert n_acc.tolist() == w["prefix_len"].tolist()
    assert (crop == 50 + 1 + n_acc).all()


# ------------------------------------------------------------------------------ sampling
def ref_sampling_probs(x, t, k, p):
    """The numpy spec of the reference test (inference/zoro-1/mlx/tests/test_tiny.py:235-246)."""
    x = x / t
    kth = np.sort(x, axis=-1)[:, -k][:, None]
    x = np.where(x < kth, -np.inf, x)
    order = np.argsort(-x, axis=-1, kind="stable")
    sx = np.take_along_axis(x, order, -1)
    e = np.exp(sx - sx.max(-1, keepdims=True))
    pr = e / e.sum(-1, keepdims=True)
    sx = np.where(np.cumsum(pr, -1) - pr >= p, -np.inf, sx)
    out = np.full_like(x, -np.inf)
    np.put_along_axis(out, order, sx, -1)
    e = np.exp(out - out.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_truncated_probs_matches_reference_spec():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(7, 1000)).astype(np.float32) * 3
    for t, k, p in [(1.0, 50, 0.95), (0.7, 20, 0.8), (1.0, 5, 1.0), (0.7, 1000, 0.95)]:
        got = A.truncated_probs(x, t, k, p)
        assert np.allclose(got, ref_sampling_probs(x, t, k, p), atol=1e-5), (t, k, p)


def test_truncated_probs_top_p_only_brute_force():
    rng = np.random.default_rng(1)
    x = (rng.normal(size=(4, 64)) * 2).astype(np.float32)
    t, p = 0.7, 0.9
    P = A.truncated_probs(x, t, 0, p)
    for r in range(4):
        l = (x[r] / np.float32(t)).astype(np.float64)
        pr = np.exp(l - l.max())
        pr /= pr.sum()
        order = np.argsort(-l)
        keep = set()
        mass = 0.0
        for i in order:  # smallest prefix whose mass reaches p
            keep.add(int(i))
            mass += pr[i]
            if mass >= p:
                break
        assert set(np.nonzero(P[r])[0].tolist()) == keep
        tot = sum(pr[i] for i in keep)
        for i in keep:
            assert abs(P[r, i] - pr[i] / tot) < 1e-12


def test_truncated_probs_mask_ban():
    x = np.zeros((1, 6), np.float32)
    x[0, 2] = 5
    P = A.truncated_probs(x, 1.0, 0, 1.0, mask_id=2)
    assert P[0, 2] == 0 and abs(P[0].sum() - 1) < 1e-12


def test_inverse_cdf():
    w = np.array([0.0, 0.25, 0.0, 0.5, 0.25])
    assert A.sample_inverse_cdf(w, 0.0)[0] == 1
    assert A.sample_inverse_cdf(w, 0.2)[0] == 1
    assert A.sample_inverse_cdf(w, 0.3)[0] == 3
    assert A.sample_inverse_cdf(w, 0.74)[0] == 3
    assert A.sample_inverse_cdf(w, 0.76)[0] == 4
    assert A.sample_inverse_cdf(w * 8, 0.999999)[0] == 4


def test_rejection_accept_closed_forms():
    V, K = 6, 3
    logits = np.zeros((1, K + 1, V), np.float32)  # P uniform on 6 tokens
    q = np.full((1, K, V), 1.0 / V)
    drafts = np.array([[0, 1, 2]])
    # p == q -> ratio 1 -> always accepted; bonus from P_K by inverse CDF
    r = A.rejection_accept(logits, q, drafts, np.full((1, K), 0.99), np.array([0.55]), temperature=1.0)
    assert r["n_acc"].tolist() == [3] and r["token"].tolist() == [3]
    # q twice p on the drafted token -> ratio 1/2: u=0.4 accepts, u=0.6 rejects
    q2 = np.full((1, K, V), 0.1)
    q2[0, :, drafts[0]] = 0.0
    for i in range(K):
        q2[0, i, drafts[0, i]] = 1.0 / 3.0
        q2[0, i] /= q2[0, i].sum()
    qd = q2[0, 0, 0]
    u = np.array([[0.4 * (1 / 6) / qd, 0.9, 0.0]])
    r = A.rejection_accept(logits, q2, drafts, u, np.array([0.0]), temperature=1.0)
    assert r["n_acc"].tolist() == [1]
    # correction comes from max(P - q, 0) at row 1: zero on the drafted token 1
    resid = np.maximum(1 / 6 - q2[0, 1], 0)
    assert resid[1] == 0 and r["token"][0] == int(np.nonzero(resid)[0][0])
    # q = 0 on a drafted token -> ratio 0 -> reject
    q3 = q.copy()
    q3[0, 0, 0] = 0
    r = A.rejection_accept(logits, q3, drafts, np.zeros((1, K)), np.array([0.0]), temperature=1.0)
    assert r["n_acc"].tolist() == [0]


def test_truncated_probs_top_k_ties_follow_topk_list():
    """With top-k the nucleus runs over exactly the k largest values (decode.py:117-122): ties at the
    k-th value beyond k do not enter the nucleus mass, but every x >= the final threshold is kept."""
    x = np.array([[3.0, 2.0, 2.0, 2.0, 0.0]], np.float32)
    # top = [3, 2]: softmax [0.731, 0.269]; mass before the 2 is 0.731 >= 0.6 -> only the 3 stays
    P = A.truncated_probs(x, 1.0, 2, 0.6)
    assert np.nonzero(P[0])[0].tolist() == [0]
    # top_p 0.8 keeps both listed values, so the threshold is 2 and all three 2s are kept
    P = A.truncated_probs(x, 1.0, 2, 0.8)
    assert np.nonzero(P[0])[0].tolist() == [0, 1, 2, 3]
    e = np.exp(np.array([3.0, 2, 2, 2]) - 3)
    assert np.allclose(P[0, :4], e / e.sum(), atol=1e-15)
    # top-k alone keeps the ties at the k-th value as well
    P = A.truncated_probs(x, 1.0, 2, 1.0)
    assert np.nonzero(P[0])[0].tolist() == [0, 1, 2, 3]


def test_apply_ban_hand_case():
    """apply_ban (decode.py:76-99): the gate compares against the probability under the *banned* row.
    p = (0.5, 0.3, 0.2); banning token 2 makes token 1's probability 0.3 / 0.8 = 0.375, so a gate of
    0.35 keeps it (taken before the ban, 0.3 < 0.35 would drop it), and a gate of 0.4 drops it."""
    x = np.log(np.array([[0.5, 0.3, 0.2]], np.float32))
    y = A.apply_ban(x, banned=(2,), gate=((1, 0.35),))
    assert np.isneginf(y[0, 2]) and np.isfinite(y[0, 1]) and y[0, 0] == x[0, 0]
    y = A.apply_ban(x, banned=(2,), gate=((1, 0.4), (0, 0.6), (7, 0.9), (0, 0.0)))
    assert np.isneginf(y[0, 1]) and np.isfinite(y[0, 0])  # p0 = 0.625 >= 0.6; id 7 and thr 0 are ignored
    assert np.allclose(A.gate_probs(A.apply_ban(x, banned=(2,)), ((1, 0.4), (0, 0.6)))[0], [0.375, 0.625])


def test_apply_ban_matches_softmax_brute_force():
    rng = np.random.default_rng(4)
    x = (rng.normal(size=(5, 40)) * 2).astype(np.float32)
    gate = ((3, 0.05), (11, 0.02), (3, 0.01))
    y = A.apply_ban(x, banned=(0, 39, 77), gate=gate)
    for r in range(5):
        row = x[r].astype(np.float64).copy()
        row[[0, 39]] = -np.inf
        p = np.exp(row - row.max())
        p /= p.sum()
        exp = row.copy()
        for tid, thr in gate:
            if p[tid] < thr:
                exp[tid] = -np.inf
        assert np.array_equal(np.isneginf(y[r]), np.isneginf(exp))
        assert np.array_equal(y[r][np.isfinite(y[r])], x[r][np.isfinite(y[r])])
