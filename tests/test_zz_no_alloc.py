"""GPU: the allocation-free greedy acceptance (trida_greedy_accept_noalloc, called through the C ABI)
returns exactly what trida_greedy_accept returns on the same inputs, on consecutive calls that share
the library's fixed device scratch (the second call smaller than the first)."""
import ctypes

import pytest
import torch

from trida_stack_amd import _lib, kernels, workloads

pytestmark = pytest.mark.gpu


def noalloc(logits, drafts, ctx_len, n_live=None):
    lib = _lib.load()
    B, R, V = logits.shape
    K = drafts.shape[1]
    dev = logits.device
    am = torch.full((B, R), -7, dtype=torch.int64, device=dev)
    n_acc = torch.full((B,), -7, dtype=torch.int32, device=dev)
    bonus = torch.full((B,), -7, dtype=torch.int64, device=dev)
    crop = torch.full((B,), -7, dtype=torch.int64, device=dev)
    dt = 0 if logits.dtype == torch.float32 else 1
    rc = lib.trida_greedy_accept_noalloc(
        logits.data_ptr(), dt, B, R, V, logits.stride(0), logits.stride(1), drafts.data_ptr(), K,
        drafts.stride(0), None if n_live is None else n_live.data_ptr(), ctx_len.data_ptr(), am.data_ptr(),
        n_acc.data_ptr(), bonus.data_ptr(), crop.data_ptr(), 0, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    _lib.check(rc, "trida_greedy_accept_noalloc")
    return am, n_acc, bonus, crop


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_greedy_accept_twice(gpu, dtype):
    # first call: batch 8 of 33 rows over the 248320 vocabulary; second: the config-1 shape (batch 1,
    # 151936); the second call leaves the first call's split results beyond its own in the array
    shapes = [dict(seed=11, batch=8, block=32, vocab=248320, ctx=2048),
              dict(seed=12, batch=1, block=32, vocab=151936, ctx=4096)]
    for sh in shapes:
        w = workloads.greedy_accept_inputs(**sh)
        logits = w["logits"].to(gpu, dtype)
        drafts, ctx = w["drafts"].to(gpu), w["ctx_len"].to(gpu)
        if dtype == torch.bfloat16:  # drafts follow the bf16 argmax so that prefixes are accepted
            am_ref = logits.float().argmax(-1)
            for b, L in enumerate(w["prefix_len"].tolist()):
                drafts[b, :L] = am_ref[b, :L]
        n_live = torch.randint(0, drafts.shape[1] + 1, (drafts.shape[0],), dtype=torch.int32).to(gpu)
        got = noalloc(logits, drafts, ctx, n_live)
        ref = kernels.greedy_accept(logits, drafts, n_live, ctx)
        torch.cuda.synchronize(gpu)
        for g, r, name in zip(got, ref, ("argmax", "n_acc", "bonus", "crop")):
            assert torch.equal(g.cpu(), r.cpu()), (sh, name)


def test_noalloc_rejects_oversized_scratch(gpu):
    lib = _lib.load()
    big = lib.trida_greedy_accept_scratch_bytes(4096, 33, 248320, 0, 0)
    assert big > 1 << 20
    x = torch.zeros(1, dtype=torch.int64, device=gpu)
    rc = lib.trida_greedy_accept_noalloc(x.data_ptr(), 0, 4096, 33, 248320, 33 * 248320, 248320, x.data_ptr(), 32, 32,
                                         None, None, None, x.data_ptr(), x.data_ptr(), x.data_ptr(), 0, None)
    assert rc == _lib.TRIDA_ERR_WORKSPACE
    assert b"scratch" in lib.trida_last_error()
