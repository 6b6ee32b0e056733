"""Torch-facing wrappers of the gfx950 kernels (C ABI in include/trida_hip.h).

Each wrapper validates shapes and dtypes, allocates outputs with torch on the input's device, and
enqueues the kernel on the current torch stream. Nothing here computes on the host: a missing library
or a CPU tensor is an error.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _need_gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("trida kernels run on the GPU only; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


class _Workspaces:
    """Device scratch per (device, name), grown on demand (never shrunk). Counter buffers are
    allocated zeroed and the kernels leave them zeroed, so they are cleared only when (re)allocated;
    scratch buffers need no initialisation."""

    def __init__(self):
        self._bufs = {}

    def get(self, dev: torch.device, name: str, nbytes: int) -> torch.Tensor:
        key = (dev.index, name)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)
            self._bufs[key] = buf
        return buf


workspaces = _Workspaces()


# --------------------------------------------------------------------------------------------------
def greedy_accept(logits: torch.Tensor, drafts: torch.Tensor, n_live: Optional[torch.Tensor] = None,
                  ctx_len: Optional[torch.Tensor] = None, *, want_argmax: bool = True, splits: int = 0):
    """Greedy acceptance over verify logits (split-V argmax + per-sequence scan, one call).

    Semantics of TridaDiffusionSampler._selfspec_step's greedy branch
    (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:906-914): per row argmax
    (first index on ties), ``match = (am[:, :K] == drafts) & (j < n_live)``, ``n_acc`` = length of the
    leading run of matches, ``bonus = am[n_acc]`` and ``crop = ctx_len + 1 + n_acc``.

    logits [B, R, V] fp32 (last dim contiguous), drafts [B, K] int64 with R >= K + 1.
    Returns (argmax [B, R] int64 or None, n_acc [B] int32, bonus [B] int64, crop [B] int64).
    """
    dev = _need_gpu(logits, drafts, n_live, ctx_len)
    if logits.dtype != torch.float32 or logits.dim() != 3 or logits.stride(2) != 1:
        raise ValueError("logits must be fp32 [B, R, V] with a contiguous last dim")
    B, R, V = logits.shape
    if drafts.dtype != torch.int64 or drafts.dim() != 2 or drafts.shape[0] != B or drafts.stride(1) != 1:
        raise ValueError("drafts must be int64 [B, K] with a contiguous last dim")
    K = drafts.shape[1]
    if R < K + 1:
        raise ValueError(f"need R >= K + 1 verify rows (R={R}, K={K})")
    if n_live is not None and (n_live.dtype != torch.int32 or n_live.shape != (B,) or not n_live.is_contiguous()):
        raise ValueError("n_live must be int32 [B]")
    if ctx_len is not None and (ctx_len.dtype != torch.int64 or ctx_len.shape != (B,) or not ctx_len.is_contiguous()):
        raise ValueError("ctx_len must be int64 [B]")
    lib = _lib.load()
    am = torch.empty((B, R), dtype=torch.int64, device=dev) if want_argmax else None
    n_acc = torch.empty(B, dtype=torch.int32, device=dev)
    bonus = torch.empty(B, dtype=torch.int64, device=dev)
    crop = torch.empty(B, dtype=torch.int64, device=dev)
    scr = workspaces.get(dev, "greedy_accept", lib.trida_greedy_accept_scratch_bytes(B, R, V, splits))
    rc = lib.trida_greedy_accept(
        logits.data_ptr(), B, R, V, logits.stride(0), logits.stride(1), _ptr(drafts), K,
        drafts.stride(0), _ptr(n_live), _ptr(ctx_len), _ptr(am), n_acc.data_ptr(), bonus.data_ptr(),
        crop.data_ptr(), scr.data_ptr(), scr.numel(), splits, _stream(dev))
    _lib.check(rc, "trida_greedy_accept")
    return am, n_acc, bonus, crop
