"""Torch-facing wrappers of the gfx950 kernels (C ABI in include/trida_hip.h).

Each wrapper validates shapes and dtypes, allocates outputs with torch on the input's device, and
enqueues the kernel on the current torch stream. Nothing here computes on the host: a missing library
or a CPU tensor is an error.
"""
from __future__ import annotations

import ctypes
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
        # buffers replaced by larger ones stay alive: a captured HIP graph may still launch kernels on them
        self._retired = []

    def get(self, dev: torch.device, name: str, nbytes: int) -> torch.Tensor:
        key = (dev.index, name)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)
            self._bufs[key] = buf
        return buf


workspaces = _Workspaces()

# Optional live timing: while TIMERS is a dict, the wrappers (and the runtime's forward) record a pair
# of events on the launching stream around their launches, keyed by name. Eager execution only.
TIMERS: Optional[dict] = None
# when not None, only these timer names record events (the rest cost nothing)
TIMER_ONLY: Optional[set] = None


class timed:
    def __init__(self, name: str):
        self.name = name
        self.ev = None

    def __enter__(self):
        if TIMERS is not None and (TIMER_ONLY is None or self.name in TIMER_ONLY):
            self.ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            self.ev[0].record()
        return self

    def __exit__(self, *exc):
        if self.ev is not None:
            self.ev[1].record()
            TIMERS.setdefault(self.name, []).append(self.ev)
        return False


def timer_means_us(timers: dict) -> dict:
    """Mean duration (us) per timer name (call after a device synchronize)."""
    return {k: sum(a.elapsed_time(b) for a, b in v) * 1e3 / len(v) for k, v in timers.items() if v}


# --------------------------------------------------------------------------------------------------
def _logit_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return 0
    if t.dtype == torch.bfloat16:
        return 1
    raise ValueError(f"logits must be fp32 or bf16 (got {t.dtype})")


def greedy_accept(logits: torch.Tensor, drafts: torch.Tensor, n_live: Optional[torch.Tensor] = None,
                  ctx_len: Optional[torch.Tensor] = None, *, want_argmax: bool = True, splits: int = 0,
                  out=None):
    """Greedy acceptance over verify logits (split-V argmax + per-sequence scan, one call).

    Semantics of TridaDiffusionSampler._selfspec_step's greedy branch
    (inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:906-914): per row argmax
    (first index on ties), ``match = (am[:, :K] == drafts) & (j < n_live)``, ``n_acc`` = length of the
    leading run of matches, ``bonus = am[n_acc]`` and ``crop = ctx_len + 1 + n_acc``.

    logits [B, R, V] fp32 or bf16 (last dim contiguous), drafts [B, K] int64 with R >= K + 1.
    out: optional preallocated (argmax [B,R] int64 or None, n_acc [B] int32, bonus [B] int64,
    crop [B] int64). Returns that tuple.
    """
    dev = _need_gpu(logits, drafts, n_live, ctx_len)
    dt = _logit_dtype(logits)
    if logits.dim() != 3 or logits.stride(2) != 1:
        raise ValueError("logits must be [B, R, V] with a contiguous last dim")
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
    if out is None:
        am = torch.empty((B, R), dtype=torch.int64, device=dev) if want_argmax else None
        out = (am, torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int64, device=dev),
               torch.empty(B, dtype=torch.int64, device=dev))
    am, n_acc, bonus, crop = out
    scr = workspaces.get(dev, "argmax", lib.trida_greedy_accept_scratch_bytes(B, R, V, dt, splits))
    rc = lib.trida_greedy_accept(
        logits.data_ptr(), dt, B, R, V, logits.stride(0), logits.stride(1), _ptr(drafts), K,
        drafts.stride(0), _ptr(n_live), _ptr(ctx_len), _ptr(am), n_acc.data_ptr(), bonus.data_ptr(),
        crop.data_ptr(), scr.data_ptr(), scr.numel(), splits, _stream(dev))
    _lib.check(rc, "trida_greedy_accept")
    return out


def row_argmax(logits: torch.Tensor, *, want_conf: bool = True, splits: int = 0, out=None):
    """Per-row argmax (first index on ties) and softmax probability of the argmax.
    logits [..., V] fp32 or bf16 with contiguous rows. Returns (argmax int64, conf fp32 or None)."""
    dev = _need_gpu(logits)
    dt = _logit_dtype(logits)
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    rows = x.shape[0]
    lib = _lib.load()
    if out is None:
        out = (torch.empty(logits.shape[:-1], dtype=torch.int64, device=dev),
               torch.empty(logits.shape[:-1], dtype=torch.float32, device=dev) if want_conf else None)
    am, conf = out
    scr = workspaces.get(dev, "argmax", lib.trida_row_argmax_scratch_bytes(rows, V, dt, splits))
    rc = lib.trida_row_argmax(x.data_ptr(), dt, rows, V, x.stride(0), am.data_ptr(), _ptr(conf), scr.data_ptr(),
                              scr.numel(), splits, _stream(dev))
    _lib.check(rc, "trida_row_argmax")
    return out


def unmask_top(argmax: torch.Tensor, conf: torch.Tensor, masked: torch.Tensor, canvas: torch.Tensor,
               count: int) -> None:
    """One denoise pass's unmasking, in place: per sequence, the `count` masked slots with the highest
    conf (ties: the lower slot first) take canvas[:, j + 1] = argmax[:, j] and leave `masked`
    (_denoise_shift_step, qwen3_5_diffusion.py:476-635, with a fixed count per pass).
    argmax [B, >= n] int64 and conf [B, >= n] fp32 with the same row stride, masked [B, n] bool,
    canvas [B, >= n + 1] int64."""
    dev = _need_gpu(argmax, conf, masked, canvas)
    B, n = masked.shape
    if masked.dtype != torch.bool or not masked.is_contiguous():
        raise ValueError("masked must be a contiguous [B, n] bool tensor")
    if argmax.dtype != torch.int64 or conf.dtype != torch.float32 or canvas.dtype != torch.int64:
        raise ValueError("argmax / canvas must be int64 and conf fp32")
    if argmax.shape[0] != B or conf.shape[0] != B or canvas.shape[0] != B or argmax.shape[1] < n \
            or conf.shape[1] < n or canvas.shape[1] < n + 1:
        raise ValueError("unmask_top: shapes do not match masked [B, n]")
    if argmax.stride() != conf.stride() or argmax.stride(1) != 1 or canvas.stride(1) != 1:
        raise ValueError("argmax and conf need the same strides and contiguous rows; canvas contiguous rows")
    rc = _lib.load().trida_unmask_top(argmax.data_ptr(), conf.data_ptr(), argmax.stride(0), masked.data_ptr(),
                                      canvas.data_ptr(), canvas.stride(0), B, n, int(count), _stream(dev))
    _lib.check(rc, "trida_unmask_top")


def canvas_advance(argmax: torch.Tensor, n_acc: torch.Tensor, canvas: torch.Tensor, verify: torch.Tensor,
                   out, mask_id: int) -> None:
    """The device-side decision of a bd_bidir_shift canvas step (selfspec_generate, decode.py:318-384):
    canvas [B, 2N-1] int64 and verify [B] uint8 are updated in place; out = (n_keep [B] int32, emit [B, N]
    int64, n_emit [B] int32, committed [B, N] int64, kind [B] int32)."""
    dev = _need_gpu(argmax, n_acc, canvas, verify)
    B, blk = canvas.shape
    N = (blk + 1) // 2
    n_keep, emit, n_emit, committed, kind = out
    if blk != 2 * N - 1 or canvas.dtype != torch.int64 or canvas.stride(1) != 1:
        raise ValueError("canvas must be int64 [B, 2N-1] with contiguous rows")
    if argmax.dtype != torch.int64 or argmax.shape[0] != B or argmax.shape[1] < blk or argmax.stride(1) != 1:
        raise ValueError("argmax must be int64 [B, >= 2N-1]")
    if verify.dtype != torch.uint8 or verify.shape != (B,) or n_acc.dtype != torch.int32 or n_acc.shape != (B,):
        raise ValueError("verify must be uint8 [B] and n_acc int32 [B]")
    for t, dt, shape in ((n_keep, torch.int32, (B,)), (emit, torch.int64, (B, N)), (n_emit, torch.int32, (B,)),
                         (committed, torch.int64, (B, N)), (kind, torch.int32, (B,))):
        if t.dtype != dt or t.shape != shape or not t.is_contiguous():
            raise ValueError("canvas_advance outputs have the wrong dtype or shape")
    rc = _lib.load().trida_canvas_advance(argmax.data_ptr(), argmax.stride(0), n_acc.data_ptr(), canvas.data_ptr(),
                                          canvas.stride(0), verify.data_ptr(), n_keep.data_ptr(), emit.data_ptr(),
                                          n_emit.data_ptr(), committed.data_ptr(), kind.data_ptr(), B, N, int(mask_id),
                                          _stream(dev))
    _lib.check(rc, "trida_canvas_advance")


def _rows2d(logits: torch.Tensor):
    """(rows, V, row stride) of logits [..., V] whose rows are evenly strided (a row-major view)."""
    V = logits.shape[-1]
    if logits.stride(-1) != 1:
        raise ValueError("logits rows must have a contiguous last dim")
    rows, rs, expect = 1, None, None
    for n, st in zip(reversed(logits.shape[:-1]), reversed(logits.stride()[:-1])):
        rows *= n
        if n == 1:
            continue
        if rs is None:
            rs = st
        elif st != expect:
            raise ValueError("logits rows must be evenly strided")
        expect = st * n
    return rows, V, (rs if rs is not None else V)


def ban_tokens(logits: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """logits[..., id] = -inf in place for every id of ids (int64 [n]), the ban of apply_ban
    (inference/zoro-1/mlx/trida_mlx/decode.py:76-99). logits fp32 or bf16 with evenly strided rows."""
    dev = _need_gpu(logits, ids)
    dt = _logit_dtype(logits)
    if ids.dtype != torch.int64 or ids.dim() != 1 or not ids.is_contiguous():
        raise ValueError("ids must be a contiguous int64 [n] tensor")
    rows, V, rs = _rows2d(logits)
    rc = _lib.load().trida_ban_tokens(logits.data_ptr(), dt, rows, V, rs, ids.data_ptr(), ids.numel(), _stream(dev))
    _lib.check(rc, "trida_ban_tokens")
    return logits


def gate_tokens(logits: torch.Tensor, ids: torch.Tensor, thr: Optional[torch.Tensor],
                raw_p: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The gate of apply_ban (decode.py:88-98), in place: per row, token ids[g] is set to -inf where its
    probability under the row's softmax, p = exp(x_id - logsumexp(x)), is below thr[g] > 0. raw_p
    [rows, n] fp32 (optional) receives every p. ids int64 [n], thr fp32 [n]. thr None (with raw_p): a
    note-only pass that writes the probabilities and leaves the logits as they are."""
    dev = _need_gpu(logits, ids, thr, raw_p)
    dt = _logit_dtype(logits)
    if thr is None and raw_p is None:
        raise ValueError("gate_tokens: thr, or raw_p for a note-only pass, is required")
    if ids.dtype != torch.int64 or ids.dim() != 1 or not ids.is_contiguous() or (thr is not None and (
            thr.dtype != torch.float32 or thr.shape != ids.shape or not thr.is_contiguous())):
        raise ValueError("ids (int64 [n]) and thr (fp32 [n]) must be contiguous and of one length")
    rows, V, rs = _rows2d(logits)
    if raw_p is not None and (raw_p.dtype != torch.float32 or raw_p.numel() < rows * ids.numel()
                              or not raw_p.is_contiguous()):
        raise ValueError("raw_p must be a contiguous fp32 tensor of rows * n elements")
    rc = _lib.load().trida_gate_tokens(logits.data_ptr(), dt, rows, V, rs, ids.data_ptr(), _ptr(thr), ids.numel(),
                                       _ptr(raw_p), _stream(dev))
    _lib.check(rc, "trida_gate_tokens")
    return logits


# --------------------------------------------------------------------------------------------------
# Sampled acceptance (temperature / top-k / top-p, speculative rejection sampling)
MAX_TOP_K = 4096


def _f32_rows(t: torch.Tensor, name: str, dims: int = 3):
    if t.dtype != torch.float32 or t.dim() != dims or t.stride(-1) != 1:
        raise ValueError(f"{name} must be fp32 with {dims} dims and a contiguous last dim")


def truncate_stats(logits: torch.Tensor, *, temperature: float, top_k: int = 0, top_p: float = 1.0,
                   ban_id: int = -1, radix_only: bool = False, want_passes: bool = False):
    """Statistics of truncated_probs (inference/zoro-1/mlx/trida_mlx/decode.py:102-130) per row of
    logits [B, R, V] fp32: m = max y (y = logit / T, ban_id at -inf), thr = smallest kept y, zk = sum of
    exp(y - m) over the kept set. Returns (m [B,R] fp32, thr [B,R] fp32, zk [B,R] fp64, status [B,R]
    int32[, passes [B,R] int32])."""
    dev = _need_gpu(logits)
    _f32_rows(logits, "logits")
    B, R, V = logits.shape
    m = torch.empty((B, R), dtype=torch.float32, device=dev)
    thr = torch.empty_like(m)
    zk = torch.empty((B, R), dtype=torch.float64, device=dev)
    st = torch.empty((B, R), dtype=torch.int32, device=dev)
    passes = torch.empty((B, R), dtype=torch.int32, device=dev) if want_passes else None
    rc = _lib.load().trida_truncate_stats(
        logits.data_ptr(), B, R, V, logits.stride(0), logits.stride(1), float(temperature), int(top_k),
        float(top_p), int(ban_id), 1 if radix_only else 0, m.data_ptr(), thr.data_ptr(), zk.data_ptr(),
        st.data_ptr(), _ptr(passes), _stream(dev))
    _lib.check(rc, "trida_truncate_stats")
    return (m, thr, zk, st, passes) if want_passes else (m, thr, zk, st)


def truncated_probs(logits: torch.Tensor, stats, *, temperature: float, ban_id: int = -1,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Truncated distributions P [B, R, V] fp32 from ``truncate_stats`` output (the probability rows the
    reference keeps as the next step's draft distributions, decode.py:354, 378)."""
    dev = _need_gpu(logits)
    _f32_rows(logits, "logits")
    B, R, V = logits.shape
    m, thr, zk = stats[0], stats[1], stats[2]
    for t, dt in ((m, torch.float32), (thr, torch.float32), (zk, torch.float64)):
        if t.dtype != dt or t.shape != (B, R) or not t.is_contiguous():
            raise ValueError("stats must be the (m, thr, zk) tensors of truncate_stats for these logits")
    if out is None:
        out = torch.empty((B, R, V), dtype=torch.float32, device=dev)
    _f32_rows(out, "out")
    rc = _lib.load().trida_truncated_probs(
        logits.data_ptr(), B, R, V, logits.stride(0), logits.stride(1), float(temperature), int(ban_id),
        m.data_ptr(), thr.data_ptr(), zk.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), _stream(dev))
    _lib.check(rc, "trida_truncated_probs")
    return out


def truncated_probs_rows(logits: torch.Tensor, stats, in_rows: torch.Tensor, out_rows: torch.Tensor, out: torch.Tensor,
                         *, temperature: float, ban_id: int = -1) -> torch.Tensor:
    """out[b, out_rows[b, j]] = truncated distribution of logits[b, in_rows[b, j]] (stats of
    ``truncate_stats`` over logits [B, R, V] fp32), for j < K; out [B, Ro, V] fp32. One launch for the
    gather / truncated_probs / scatter that keeps a draft pass's unmasked slots' q rows. Indices outside
    [0, R) / [0, Ro) skip their row."""
    dev = _need_gpu(logits, in_rows, out_rows, out)
    _f32_rows(logits, "logits")
    _f32_rows(out, "out")
    B, R, V = logits.shape
    m, thr, zk = stats[0], stats[1], stats[2]
    for t, dt in ((m, torch.float32), (thr, torch.float32), (zk, torch.float64)):
        if t.dtype != dt or t.shape != (B, R) or not t.is_contiguous():
            raise ValueError("stats must be the (m, thr, zk) tensors of truncate_stats for these logits")
    for t, n in ((in_rows, "in_rows"), (out_rows, "out_rows")):
        if t.dtype != torch.int64 or t.dim() != 2 or t.shape[0] != B or not t.is_contiguous():
            raise ValueError(f"{n} must be int64 [B, K] contiguous")
    if in_rows.shape != out_rows.shape or out.shape[0] != B or out.shape[2] != V:
        raise ValueError("in_rows / out_rows / out shapes disagree")
    rc = _lib.load().trida_truncated_probs_rows(
        logits.data_ptr(), B, R, V, logits.stride(0), logits.stride(1), float(temperature), int(ban_id),
        m.data_ptr(), thr.data_ptr(), zk.data_ptr(), in_rows.data_ptr(), out_rows.data_ptr(), in_rows.shape[1],
        out.data_ptr(), out.shape[1], out.stride(0), out.stride(1), _stream(dev))
    _lib.check(rc, "trida_truncated_probs_rows")
    return out


def gather_rows(src: torch.Tensor, rows: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[b, k] = fp32(src[b, rows[b, k]]) for src [B, R, V] bf16 or fp32 (contiguous last dim), rows int64
    [B, K]: a row gather and the widening to fp32 in one pass. Indices outside [0, R) skip their row."""
    dev = _need_gpu(src, rows, out)
    dt = _logit_dtype(src)
    if src.dim() != 3 or src.stride(2) != 1:
        raise ValueError("src must be [B, R, V] with a contiguous last dim")
    B, R, V = src.shape
    if rows.dtype != torch.int64 or rows.dim() != 2 or rows.shape[0] != B or not rows.is_contiguous():
        raise ValueError("rows must be int64 [B, K] contiguous")
    K_ = rows.shape[1]
    if out is None:
        out = torch.empty((B, K_, V), dtype=torch.float32, device=dev)
    _f32_rows(out, "out")
    if out.shape != (B, K_, V):
        raise ValueError("out must be [B, K, V] fp32")
    rc = _lib.load().trida_gather_rows(src.data_ptr(), dt, B, R, V, src.stride(0), src.stride(1), rows.data_ptr(),
                                       K_, out.data_ptr(), out.stride(0), out.stride(1), _stream(dev))
    _lib.check(rc, "trida_gather_rows")
    return out


def sample_rows(logits: torch.Tensor, stats, u: torch.Tensor, *, temperature: float, ban_id: int = -1,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One token per row of logits [..., V] fp32 (contiguous rows) from the truncated distribution of
    ``truncate_stats`` output (inverse CDF in vocabulary order at u, one uniform per row)."""
    dev = _need_gpu(logits, u, out)
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.dtype != torch.float32 or x.stride(1) != 1:
        raise ValueError("logits must be fp32 with contiguous rows")
    rows = x.shape[0]
    m, thr, zk = (t.reshape(-1) for t in stats[:3])
    for t, dt in ((m, torch.float32), (thr, torch.float32), (zk, torch.float64)):
        if t.dtype != dt or t.numel() != rows or not t.is_contiguous():
            raise ValueError("stats must be the (m, thr, zk) tensors of truncate_stats for these rows")
    if u.dtype != torch.float32 or u.numel() != rows or not u.is_contiguous():
        raise ValueError("u must be fp32 with one uniform per row")
    if out is None:
        out = torch.empty(logits.shape[:-1], dtype=torch.int64, device=dev)
    lib = _lib.load()
    scr = workspaces.get(dev, "draw", lib.trida_sample_rows_scratch_bytes(rows, V))
    rc = lib.trida_sample_rows(x.data_ptr(), rows, V, x.stride(0), float(temperature), int(ban_id), m.data_ptr(),
                               thr.data_ptr(), zk.data_ptr(), u.data_ptr(), out.data_ptr(), scr.data_ptr(), scr.numel(),
                               _stream(dev))
    _lib.check(rc, "trida_sample_rows")
    return out


def sample_accept(p_logits: torch.Tensor, q_probs: Optional[torch.Tensor], drafts: torch.Tensor,
                  u_accept: Optional[torch.Tensor], u_sample: torch.Tensor, *, temperature: float,
                  top_k: int = 0, top_p: float = 1.0, ban_id: int = -1, n_live: Optional[torch.Tensor] = None,
                  ctx_len: Optional[torch.Tensor] = None, want_ratio: bool = False, out=None):
    """Sampled acceptance of a verify pass (selfspec_generate's sampled verify,
    inference/zoro-1/mlx/trida_mlx/decode.py:333-354): per draft ratio P_i(d_i) / q_i(d_i), accepted while
    ``ratio >= 1 or u < ratio``; the correction (or, when every draft is accepted, the bonus) is drawn by
    inverse CDF at ``u_sample`` from max(0, P_a - q_a) (P_a when that is empty) or P_K.

    p_logits [B, R, V] fp32, q_probs [B, K, V] fp32, drafts [B, K] int64, u_accept [B, K] fp32,
    u_sample [B] fp32. Returns (n_acc [B] int32, token [B] int64, crop [B] int64, ratio [B, K] fp64 or
    None, status [B] int32)."""
    dev = _need_gpu(p_logits, q_probs, drafts, u_accept, u_sample, n_live, ctx_len)
    _f32_rows(p_logits, "p_logits")
    B, R, V = p_logits.shape
    if drafts.dtype != torch.int64 or drafts.dim() != 2 or drafts.shape[0] != B or (
            drafts.shape[1] > 0 and drafts.stride(1) != 1):
        raise ValueError("drafts must be int64 [B, K] with a contiguous last dim")
    K = drafts.shape[1]
    if K:
        _f32_rows(q_probs, "q_probs")
        if q_probs.shape != (B, K, V):
            raise ValueError(f"q_probs must be [B, K, V] = {(B, K, V)}")
        _f32_rows(u_accept, "u_accept", 2)
        if u_accept.shape != (B, K):
            raise ValueError("u_accept must be [B, K]")
    if u_sample.dtype != torch.float32 or u_sample.shape != (B,) or not u_sample.is_contiguous():
        raise ValueError("u_sample must be fp32 [B]")
    if n_live is not None and (n_live.dtype != torch.int32 or n_live.shape != (B,) or not n_live.is_contiguous()):
        raise ValueError("n_live must be int32 [B]")
    if ctx_len is not None and (ctx_len.dtype != torch.int64 or ctx_len.shape != (B,) or not ctx_len.is_contiguous()):
        raise ValueError("ctx_len must be int64 [B]")
    lib = _lib.load()
    if out is None:
        out = (torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int64, device=dev),
               torch.empty(B, dtype=torch.int64, device=dev),
               torch.empty((B, K), dtype=torch.float64, device=dev) if want_ratio else None,
               torch.empty(B, dtype=torch.int32, device=dev))
    n_acc, token, crop, ratio, status = out
    scr = workspaces.get(dev, "sample", lib.trida_sample_accept_scratch_bytes(B, R, V, K))
    rc = lib.trida_sample_accept(
        p_logits.data_ptr(), B, R, V, p_logits.stride(0), p_logits.stride(1), _ptr(q_probs),
        q_probs.stride(0) if K else 0, q_probs.stride(1) if K else 0, drafts.data_ptr(), K,
        drafts.stride(0) if K else 0,
        _ptr(n_live), _ptr(u_accept), u_accept.stride(0) if K else 0, u_sample.data_ptr(), _ptr(ctx_len),
        float(temperature), int(top_k), float(top_p), int(ban_id), n_acc.data_ptr(), token.data_ptr(),
        crop.data_ptr(), _ptr(ratio), status.data_ptr(), scr.data_ptr(), scr.numel(), _stream(dev))
    _lib.check(rc, "trida_sample_accept")
    return out


# --------------------------------------------------------------------------------------------------
# GDN (gated delta net) layer pieces
def _bf16(t: torch.Tensor, name: str):
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bf16 (got {t.dtype})")


def _f32(t: torch.Tensor, name: str):
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be fp32 (got {t.dtype})")


def _i32(t: Optional[torch.Tensor], name: str, n: Optional[int] = None):
    """A contiguous int32 index vector (optionally of n entries), or None."""
    if t is None:
        return None
    if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous() or (n is not None and t.numel() != n):
        raise ValueError(f"{name} must be a contiguous int32 vector" + (f" of {n} entries" if n is not None else ""))
    return t


def _packed(cu_seqlens: Optional[torch.Tensor], max_rows: Optional[int]):
    """(B, T) of a packed ragged batch: B sequences, T an upper bound of their rows."""
    _i32(cu_seqlens, "cu_seqlens")
    if max_rows is None or int(max_rows) < 1:
        raise ValueError("a packed batch (cu_seqlens) needs max_rows >= 1, an upper bound of every sequence's rows")
    return cu_seqlens.numel() - 1, int(max_rows)


# The kernels take the pool / ring indices and cu_seqlens as given (as the reference's kernels do): an entry
# out of range would address memory outside the pools. Outside graph capture the wrappers read them back
# (one small device-to-host copy) and refuse such entries before any launch; under capture they are trusted.
def _checkable(t: Optional[torch.Tensor]) -> bool:
    return t is not None and t.numel() > 0 and not torch.cuda.is_current_stream_capturing()


def _idx_range(idx: Optional[torch.Tensor], rows: int, name: str, distinct: bool = False) -> None:
    """Every entry of the index vector in [0, rows) (and pairwise distinct when asked)."""
    if not _checkable(idx):
        return
    v = idx.cpu()
    lo, hi = int(v.min()), int(v.max())
    if lo < 0 or hi >= rows:
        raise ValueError(f"{name}: entries must lie in [0, {rows}) (got {lo} .. {hi})")
    if distinct and torch.unique(v).numel() != v.numel():
        raise ValueError(f"{name}: entries must be distinct when the pool is written in place")


def _seqlens_range(cu_seqlens: Optional[torch.Tensor], total: int) -> None:
    """cu_seqlens starts at >= 0, never decreases and ends within the total rows of the packed tensors."""
    if not _checkable(cu_seqlens):
        return
    v = cu_seqlens.cpu().long()
    if int(v[0]) < 0 or int(v[-1]) > total or bool((v[1:] < v[:-1]).any()):
        raise ValueError(f"cu_seqlens must be non-decreasing within [0, {total}] (got {v.tolist()[:8]} ...)")


def gdn_prep(x: torch.Tensor, window: torch.Tensor, conv_w: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
             A_log: torch.Tensor, dt_bias: torch.Tensor, *, Hk: int, Hv: int, Dk: int, Dv: int,
             window_out: Optional[torch.Tensor] = None, pre_out: Optional[torch.Tensor] = None, out=None,
             conv_bias: Optional[torch.Tensor] = None, win_idx: Optional[torch.Tensor] = None,
             pre_idx: Optional[torch.Tensor] = None, cu_seqlens: Optional[torch.Tensor] = None,
             max_rows: Optional[int] = None):
    """Conv + SiLU + split + l2norm(q, k) + gates for a block of rows (one launch).

    x [B, T, C] bf16 (last dim contiguous, C = 2*Hk*Dk + Hv*Dv; batch / row strides may be larger),
    window [B, Kc-1, C] bf16, conv_w [C, Kc] bf16, a, b [B, T, Hv] bf16 (last dim contiguous),
    A_log, dt_bias [Hv] fp32. Returns q, k [B,T,Hk,Dk] bf16, v [B,T,Hv,Dv] bf16, g, beta [B,T,Hv] fp32.
    window_out (optional, [B, Kc-1, C], not aliasing window) receives the last Kc-1 rows of
    [window ++ x] (the causal-prefill conv state). pre_out (optional, contiguous [B, T, C]) receives a
    copy of x: the pre-conv rows a rollback rebuilds the window from.

    Pool and packed forms (the vLLM conv call's arguments): conv_bias [C] bf16; win_idx int32 [B] picks
    each sequence's window row of a [rows, Kc-1, C] pool (window_out is then a pool too); pre_idx
    int32 [B] its pre_out slot of a [slots, T, C] pool; cu_seqlens int32 [B + 1] with max_rows packs the
    batch: x [total, C], a, b [total, Hv] and the outputs [total, ...]."""
    dev = _need_gpu(x, window, conv_w, a, b, A_log, dt_bias, window_out, pre_out, conv_bias, win_idx, pre_idx,
                    cu_seqlens)
    for t, n in ((x, "x"), (window, "window"), (conv_w, "conv_w"), (a, "a"), (b, "b")):
        _bf16(t, n)
    _f32(A_log, "A_log")
    _f32(dt_bias, "dt_bias")
    packed = cu_seqlens is not None
    if packed:
        B, T = _packed(cu_seqlens, max_rows)
        if x.dim() != 2 or a.dim() != 2:
            raise ValueError("a packed batch takes x [total, C] and a, b [total, Hv]")
        rows, C = x.shape
        lead = (rows,)
        x_sb, x_st = 0, x.stride(0)
        ab_sb, ab_st = 0, a.stride(0)
    else:
        B, T, C = x.shape
        lead = (B, T)
        x_sb, x_st = x.stride(0), x.stride(1)
        ab_sb, ab_st = a.stride(0), a.stride(1)
    Kc = conv_w.shape[1]
    if C != 2 * Hk * Dk + Hv * Dv or conv_w.shape != (C, Kc) or not conv_w.is_contiguous():
        raise ValueError("x / conv_w do not match the head geometry")
    win_rows = window.shape[0] if win_idx is not None else B
    if x.stride(-1) != 1 or window.shape != (win_rows, Kc - 1, C) or not window.is_contiguous():
        raise ValueError("x must have a contiguous last dim and window be contiguous [B (or pool rows), Kc-1, C]")
    if a.shape != lead + (Hv,) or b.shape != a.shape or a.stride() != b.stride() or a.stride(-1) != 1:
        raise ValueError("a and b must be [..., Hv] like x's rows, with identical strides and a contiguous last dim")
    _i32(win_idx, "win_idx", B)
    _i32(pre_idx, "pre_idx", B)
    if conv_bias is not None:
        _bf16(conv_bias, "conv_bias")
        if conv_bias.shape != (C,) or not conv_bias.is_contiguous():
            raise ValueError("conv_bias must be contiguous [C]")
    if window_out is not None and (window_out.shape[1:] != window.shape[1:] or not window_out.is_contiguous()
                                   or (win_idx is None and window_out.shape != window.shape)
                                   or window_out.data_ptr() == window.data_ptr()):
        raise ValueError("window_out must be a separate contiguous [B (or pool rows), Kc-1, C] buffer")
    if pre_out is not None:
        _bf16(pre_out, "pre_out")
        slots = pre_out.shape[0] if pre_idx is not None else B
        if pre_out.shape != (slots, T, C) or not pre_out.is_contiguous() or pre_out.data_ptr() == x.data_ptr():
            raise ValueError("pre_out must be a separate contiguous [B (or pool slots), T, C] buffer")
    _idx_range(win_idx, min(win_rows, window_out.shape[0]) if window_out is not None else win_rows, "win_idx")
    if pre_out is not None:
        _idx_range(pre_idx, pre_out.shape[0], "pre_idx")
    if packed:
        _seqlens_range(cu_seqlens, lead[0])
    if out is None:
        q = torch.empty(lead + (Hk, Dk), dtype=torch.bfloat16, device=dev)
        k = torch.empty_like(q)
        v = torch.empty(lead + (Hv, Dv), dtype=torch.bfloat16, device=dev)
        g = torch.empty(lead + (Hv,), dtype=torch.float32, device=dev)
        beta = torch.empty_like(g)
    else:
        q, k, v, g, beta = out
        if q.shape != lead + (Hk, Dk) or k.shape != q.shape or v.shape != lead + (Hv, Dv) or g.shape != lead + (Hv,) \
                or beta.shape != g.shape or not all(t.is_contiguous() for t in out):
            raise ValueError("gdn_prep: out buffers have the wrong shape")
    rc = _lib.load().trida_gdn_prep(
        x.data_ptr(), window.data_ptr(), conv_w.data_ptr(), a.data_ptr(), b.data_ptr(),
        A_log.contiguous().data_ptr(), dt_bias.contiguous().data_ptr(), q.data_ptr(), k.data_ptr(),
        v.data_ptr(), g.data_ptr(), beta.data_ptr(), _ptr(window_out), _ptr(pre_out), B, T, Kc, Hk, Hv, Dk, Dv,
        x_sb, x_st, ab_sb, ab_st, _ptr(conv_bias), _ptr(win_idx), _ptr(pre_idx), _ptr(cu_seqlens), _stream(dev))
    _lib.check(rc, "trida_gdn_prep")
    return q, k, v, g, beta


def _state_pool(state: torch.Tensor, B: int, Hv: int, Dv: int, Dk: int, state_idx: Optional[torch.Tensor]):
    _i32(state_idx, "state_idx", B)
    rows = state.shape[0] if state_idx is not None else B
    if state.shape != (rows, Hv, Dv, Dk) or not state.is_contiguous():
        raise ValueError(f"state must be contiguous [B (or pool rows), Hv, Dv, Dk] = {(rows, Hv, Dv, Dk)}")


def _ring(inter: Optional[torch.Tensor], inter_idx: Optional[torch.Tensor], cache_steps: Optional[int], B: int,
          Hv: int, Dv: int, Dk: int) -> int:
    """cache_steps of an intermediate-state ring inter [rows, cache_steps, Hv, Dv, Dk] fp32 (0 without)."""
    if inter is None:
        if inter_idx is not None:
            raise ValueError("inter_idx without inter")
        return 0
    _f32(inter, "inter")
    steps = inter.shape[1] if cache_steps is None else int(cache_steps)
    rows = inter.shape[0] if inter_idx is not None else B
    if inter.dim() != 5 or inter.shape != (rows, steps, Hv, Dv, Dk) or not inter.is_contiguous() or steps < 1:
        raise ValueError(f"inter must be contiguous [B (or ring rows), cache_steps, Hv, Dv, Dk] fp32")
    _i32(inter_idx, "inter_idx", B)
    return steps


def gdr_recurrent(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                  state: torch.Tensor, *, causal_mode: int = 1, num_clean: Optional[int] = None,
                  state_out: Optional[torch.Tensor] = None, want_clean: bool = False,
                  scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                  cu_seqlens: Optional[torch.Tensor] = None, max_rows: Optional[int] = None,
                  state_idx: Optional[torch.Tensor] = None, inter: Optional[torch.Tensor] = None,
                  inter_idx: Optional[torch.Tensor] = None, cache_steps: Optional[int] = None):
    """Gated delta rule over T rows with the block-causal readout (one launch).

    q, k [B,T,Hk,Dk] bf16, v [B,T,Hv,Dv] bf16, g (log decay), beta [B,T,Hv] fp32, state [B,Hv,Dv,Dk]
    fp32 (read only unless passed again as state_out). causal_mode 2 with num_clean: rows >= num_clean
    read the block-end state. Returns (out [B,T,Hv,Dv] bf16, state_clean or None).

    Pool, ring and packed forms (fused_recurrent_block_causal_gated_delta_rule[_packed]'s arguments):
    state_idx int32 [B] picks each sequence's row of a state pool [rows, Hv, Dv, Dk] (read, and written
    when state_out is the pool); inter [rows, cache_steps, Hv, Dv, Dk] fp32 with inter_idx int32 [B]
    receives the state after rows 0..j (j < cache_steps) of each sequence; cu_seqlens int32 [B + 1] with
    max_rows packs the batch: q, k [total, Hk, Dk], v [total, Hv, Dv], g, beta [total, Hv], out
    [total, Hv, Dv]."""
    dev = _need_gpu(q, k, v, g, beta, state, state_out, cu_seqlens, state_idx, inter, inter_idx)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _bf16(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    for t, n in ((g, "g"), (beta, "beta"), (state, "state")):
        _f32(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    Hk, Dk = k.shape[-2:]
    Hv, Dv = v.shape[-2:]
    if cu_seqlens is not None:
        B, T = _packed(cu_seqlens, max_rows)
        if k.dim() != 3:
            raise ValueError("a packed batch takes q, k [total, Hk, Dk], v [total, Hv, Dv], g, beta [total, Hv]")
        lead = (k.shape[0],)
    else:
        B, T = k.shape[:2]
        lead = (B, T)
    if q.shape != k.shape or v.shape[:-2] != lead or g.shape != lead + (Hv,) or beta.shape != g.shape:
        raise ValueError("q/k/v/g/beta shapes disagree")
    _state_pool(state, B, Hv, Dv, Dk, state_idx)
    if state_out is not None and (state_out.shape != state.shape or state_out.dtype != torch.float32
                                  or not state_out.is_contiguous()):
        raise ValueError("state_out must match state")
    steps = _ring(inter, inter_idx, cache_steps, B, Hv, Dv, Dk)
    _idx_range(state_idx, state.shape[0], "state_idx",
               distinct=state_out is not None and state_out.data_ptr() == state.data_ptr())
    if inter is not None:
        _idx_range(inter_idx, inter.shape[0], "inter_idx")
    if cu_seqlens is not None:
        _seqlens_range(cu_seqlens, lead[0])
    nc = T if num_clean is None else int(num_clean)
    if out is None:
        out = torch.empty(lead + (Hv, Dv), dtype=torch.bfloat16, device=dev)
    elif out.shape != lead + (Hv, Dv) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("gdr_recurrent: out must be contiguous bf16 like v")
    clean = torch.empty((B, Hv, Dv, Dk), dtype=torch.float32, device=dev) if want_clean else None
    sc = Dk ** -0.5 if scale is None else float(scale)
    rc = _lib.load().trida_gdr_recurrent(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), state.data_ptr(),
        out.data_ptr(), _ptr(state_out), _ptr(clean), B, T, Hk, Hv, Dk, Dv, causal_mode, nc, sc,
        _ptr(cu_seqlens), _ptr(state_idx), _ptr(inter), _ptr(inter_idx), steps, _stream(dev))
    _lib.check(rc, "trida_gdr_recurrent")
    return out, clean


def gdr_recurrent_gnorm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                        state: torch.Tensor, z: torch.Tensor, gnorm_w: torch.Tensor, u_frag: torch.Tensor,
                        ss_parts: torch.Tensor, *, causal_mode: int = 1, num_clean: Optional[int] = None,
                        state_out: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gdr_recurrent (contiguous form, B * T <= 48, T <= 40) that also leaves the gated RMSNorm's inputs for
    ws_gemm_headnorm: u_frag (ws_frag_numel(Hv * Dv) bf16) = bf16(bf16(o) * gnorm_w * silu(z)) in fragment
    order and ss_parts fp32 [B * T, Hv, Dv / 8] = the sums of bf16(o)^2 over each 8 columns. z [B * T,
    >= Hv * Dv] bf16 with contiguous rows; gnorm_w [Dv] bf16. Returns out [B, T, Hv, Dv] bf16 (o)."""
    dev = _need_gpu(q, k, v, g, beta, state, z, gnorm_w, u_frag, ss_parts, state_out, out)
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (gnorm_w, "gnorm_w")):
        _bf16(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    for t, n in ((g, "g"), (beta, "beta"), (state, "state"), (ss_parts, "ss_parts")):
        _f32(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[-2:]
    if q.shape != k.shape or v.shape[:2] != (B, T) or g.shape != (B, T, Hv) or beta.shape != g.shape \
            or state.shape != (B, Hv, Dv, Dk):
        raise ValueError("q/k/v/g/beta/state shapes disagree")
    _bf16(z, "z")
    if z.dim() != 2 or z.shape[0] != B * T or z.shape[1] < Hv * Dv or z.stride(1) != 1 or gnorm_w.numel() != Dv:
        raise ValueError("gdr_recurrent_gnorm: z [B T, >= Hv Dv] with contiguous rows and gnorm_w [Dv]")
    _frag_buf(u_frag, Hv * Dv, "u_frag")
    if ss_parts.numel() < B * T * Hv * (Dv // 8):
        raise ValueError("gdr_recurrent_gnorm: ss_parts needs B T Hv Dv / 8 floats")
    if state_out is not None and (state_out.shape != state.shape or state_out.dtype != torch.float32
                                  or not state_out.is_contiguous()):
        raise ValueError("state_out must match state")
    if out is None:
        out = torch.empty(B, T, Hv, Dv, dtype=torch.bfloat16, device=dev)
    elif out.shape != (B, T, Hv, Dv) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("gdr_recurrent_gnorm: out must be contiguous bf16 like v")
    nc = T if num_clean is None else int(num_clean)
    sc = Dk ** -0.5 if scale is None else float(scale)
    rc = _lib.load().trida_gdr_recurrent_gnorm(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), state.data_ptr(), out.data_ptr(),
        _ptr(state_out), None, B, T, Hk, Hv, Dk, Dv, causal_mode, nc, sc, z.data_ptr(), z.stride(0),
        gnorm_w.data_ptr(), u_frag.data_ptr(), ss_parts.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_gdr_recurrent_gnorm")
    return out


def gdn_fused_layer(x: torch.Tensor, window: torch.Tensor, conv_w: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
                    A_log: torch.Tensor, dt_bias: torch.Tensor, state: torch.Tensor, *, Hk: int, Hv: int, Dk: int,
                    Dv: int, causal_mode: int = 1, num_clean: Optional[int] = None,
                    state_out: Optional[torch.Tensor] = None, want_clean: bool = False,
                    rows_out: Optional[tuple] = None, pre_out: Optional[torch.Tensor] = None,
                    window_out: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                    out: Optional[torch.Tensor] = None, conv_bias: Optional[torch.Tensor] = None,
                    win_idx: Optional[torch.Tensor] = None, state_idx: Optional[torch.Tensor] = None,
                    inter: Optional[torch.Tensor] = None, inter_idx: Optional[torch.Tensor] = None,
                    cache_steps: Optional[int] = None, pre_idx: Optional[torch.Tensor] = None):
    """The GDN layer's conv + prep + recurrence + readout for a block of T <= 64 rows in one launch
    (fused_selfspec_gdn_layer, qwen3_5_diffusion.py:2207-2221); bit-identical to gdn_prep followed by
    gdr_recurrent. Inputs as gdn_prep plus state [B, Hv, Dv, Dk] fp32. Optional outputs:
    rows_out = (k [B,T,Hk,Dk] bf16, v [B,T,Hv,Dv] bf16, g, beta [B,T,Hv] fp32) for a rollback,
    pre_out [B, T, C] bf16 (raw pre-conv rows), window_out [B, Kc-1, C] (not aliasing window).
    The vLLM call's pool / ring arguments (conv_bias, win_idx, state_idx = ssm_idx, inter / inter_idx /
    cache_steps, pre_idx = slot_idx) have the meanings of gdn_prep and gdr_recurrent.
    Returns (out [B,T,Hv,Dv] bf16, state_clean or None)."""
    dev = _need_gpu(x, window, conv_w, a, b, A_log, dt_bias, state, state_out, out, pre_out, window_out, conv_bias,
                    win_idx, state_idx, inter, inter_idx, pre_idx)
    for t, n in ((x, "x"), (window, "window"), (conv_w, "conv_w"), (a, "a"), (b, "b")):
        _bf16(t, n)
    for t, n in ((A_log, "A_log"), (dt_bias, "dt_bias"), (state, "state")):
        _f32(t, n)
    B, T, C = x.shape
    Kc = conv_w.shape[1]
    if C != 2 * Hk * Dk + Hv * Dv or conv_w.shape != (C, Kc) or not conv_w.is_contiguous():
        raise ValueError("x / conv_w do not match the head geometry")
    win_rows = window.shape[0] if win_idx is not None else B
    if x.stride(2) != 1 or window.shape != (win_rows, Kc - 1, C) or not window.is_contiguous():
        raise ValueError("x must have a contiguous last dim and window be contiguous [B (or pool rows), Kc-1, C]")
    if a.shape != (B, T, Hv) or b.shape != (B, T, Hv) or a.stride() != b.stride() or a.stride(2) != 1:
        raise ValueError("a and b must be [B, T, Hv] with identical strides and a contiguous last dim")
    _i32(win_idx, "win_idx", B)
    _i32(pre_idx, "pre_idx", B)
    _state_pool(state, B, Hv, Dv, Dk, state_idx)
    if state_out is not None and (state_out.shape != state.shape or state_out.dtype != torch.float32
                                  or not state_out.is_contiguous()):
        raise ValueError("state_out must match state")
    steps = _ring(inter, inter_idx, cache_steps, B, Hv, Dv, Dk)
    if conv_bias is not None:
        _bf16(conv_bias, "conv_bias")
        if conv_bias.shape != (C,) or not conv_bias.is_contiguous():
            raise ValueError("conv_bias must be contiguous [C]")
    if window_out is not None and (window_out.shape[1:] != window.shape[1:] or not window_out.is_contiguous()
                                   or (win_idx is None and window_out.shape != window.shape)
                                   or window_out.data_ptr() == window.data_ptr()):
        raise ValueError("window_out must be a separate contiguous [B (or pool rows), Kc-1, C] buffer")
    if pre_out is not None:
        slots = pre_out.shape[0] if pre_idx is not None else B
        if pre_out.shape != (slots, T, C) or pre_out.dtype != torch.bfloat16 or not pre_out.is_contiguous():
            raise ValueError("pre_out must be contiguous bf16 [B (or pool slots), T, C]")
    _idx_range(win_idx, min(win_rows, window_out.shape[0]) if window_out is not None else win_rows, "win_idx")
    if pre_out is not None:
        _idx_range(pre_idx, pre_out.shape[0], "pre_idx")
    _idx_range(state_idx, state.shape[0], "state_idx",
               distinct=state_out is not None and state_out.data_ptr() == state.data_ptr())
    if inter is not None:
        _idx_range(inter_idx, inter.shape[0], "inter_idx")
    kr = vr = gr = br = None
    if rows_out is not None:
        kr, vr, gr, br = rows_out
        if kr.shape != (B, T, Hk, Dk) or vr.shape != (B, T, Hv, Dv) or gr.shape != (B, T, Hv) \
                or br.shape != gr.shape or not all(t.is_contiguous() for t in rows_out):
            raise ValueError("gdn_fused_layer: rows_out buffers have the wrong shape")
    nc = T if num_clean is None else int(num_clean)
    if out is None:
        out = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev)
    elif out.shape != (B, T, Hv, Dv) or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("gdn_fused_layer: out must be contiguous bf16 [B, T, Hv, Dv]")
    clean = torch.empty((B, Hv, Dv, Dk), dtype=torch.float32, device=dev) if want_clean else None
    sc = Dk ** -0.5 if scale is None else float(scale)
    rc = _lib.load().trida_gdn_fused_layer(
        x.data_ptr(), window.data_ptr(), conv_w.data_ptr(), a.data_ptr(), b.data_ptr(),
        A_log.contiguous().data_ptr(), dt_bias.contiguous().data_ptr(), state.data_ptr(), out.data_ptr(),
        _ptr(state_out), _ptr(clean), _ptr(kr), _ptr(vr), _ptr(gr), _ptr(br), _ptr(pre_out), _ptr(window_out),
        B, T, Kc, Hk, Hv, Dk, Dv, x.stride(0), x.stride(1), a.stride(0), a.stride(1), causal_mode, nc, sc,
        _ptr(conv_bias), _ptr(win_idx), _ptr(state_idx), _ptr(inter), _ptr(inter_idx), steps, _ptr(pre_idx),
        _stream(dev))
    _lib.check(rc, "trida_gdn_fused_layer")
    return out, clean


def gdr_block_bidir(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                    state: torch.Tensor, *, block_size: int, state_out: Optional[torch.Tensor] = None,
                    scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block-bidirectional gated delta rule (the training research readout of
    train/models/hybrid.py:461-536) over blocks of block_size rows: each row reads out the mean of the
    causal readout and a reversed within-block scan from the block-entry state. Same shapes as
    gdr_recurrent. Returns out [B, T, Hv, Dv] bf16."""
    dev = _need_gpu(q, k, v, g, beta, state, state_out, out)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _bf16(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    for t, n in ((g, "g"), (beta, "beta"), (state, "state")):
        _f32(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2], v.shape[3]
    if q.shape != k.shape or v.shape[:2] != (B, T) or g.shape != (B, T, Hv) or beta.shape != g.shape:
        raise ValueError("q/k/v/g/beta shapes disagree")
    if state.shape != (B, Hv, Dv, Dk):
        raise ValueError(f"state must be [B, Hv, Dv, Dk] = {(B, Hv, Dv, Dk)}")
    if state_out is not None and (state_out.shape != state.shape or state_out.dtype != torch.float32
                                  or not state_out.is_contiguous()):
        raise ValueError("state_out must match state")
    if out is None:
        out = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev)
    sc = Dk ** -0.5 if scale is None else float(scale)
    rc = _lib.load().trida_gdr_block_bidir(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                           state.data_ptr(), out.data_ptr(), _ptr(state_out), B, T, Hk, Hv, Dk, Dv,
                                           int(block_size), sc, _stream(dev))
    _lib.check(rc, "trida_gdr_block_bidir")
    return out


def gdr_chunk(q: Optional[torch.Tensor], k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
              state: torch.Tensor, *, causal_mode: int = 1, num_clean: Optional[int] = None,
              state_out: Optional[torch.Tensor] = None, n_keep: Optional[torch.Tensor] = None,
              want_out: bool = True, scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
              cu_seqlens: Optional[torch.Tensor] = None, max_rows: Optional[int] = None,
              state_idx: Optional[torch.Tensor] = None):
    """Gated delta rule in the chunked WY / UT form on MFMA (chunks of 64 rows; one fused launch for
    T <= 64). Same shapes and readout as gdr_recurrent. n_keep (int32 [B] or [seq_mod] with B a multiple):
    state_out holds the state after the first n_keep[b] rows (the rollback). want_out=False skips the
    readout (q may be None). cu_seqlens (int32 [B + 1]) with max_rows packs a ragged batch ([total, ...]
    rows) and state_idx (int32 [B]) picks each sequence's row of a state pool, as in gdr_recurrent.
    Returns out (or None)."""
    dev = _need_gpu(q, k, v, g, beta, state, state_out, n_keep, out, cu_seqlens, state_idx)
    for t, n in ((k, "k"), (v, "v")) + (((q, "q"),) if q is not None else ()):
        _bf16(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    for t, n in ((g, "g"), (beta, "beta"), (state, "state")):
        _f32(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    Hk, Dk = k.shape[-2:]
    Hv, Dv = v.shape[-2:]
    if cu_seqlens is not None:
        B, T = _packed(cu_seqlens, max_rows)
        if k.dim() != 3:
            raise ValueError("a packed batch takes k [total, Hk, Dk], v [total, Hv, Dv], g, beta [total, Hv]")
        lead = (k.shape[0],)
    else:
        B, T = k.shape[:2]
        lead = (B, T)
    if (q is not None and q.shape != k.shape) or v.shape[:-2] != lead or g.shape != lead + (Hv,) \
            or beta.shape != g.shape:
        raise ValueError("q/k/v/g/beta shapes disagree")
    _state_pool(state, B, Hv, Dv, Dk, state_idx)
    if state_out is not None and (state_out.shape != state.shape or state_out.dtype != torch.float32
                                  or not state_out.is_contiguous()):
        raise ValueError("state_out must match state")
    _idx_range(state_idx, state.shape[0], "state_idx",
               distinct=state_out is not None and state_out.data_ptr() == state.data_ptr())
    if cu_seqlens is not None:
        _seqlens_range(cu_seqlens, lead[0])
    seq_mod = 0
    if n_keep is not None:
        if n_keep.dtype != torch.int32 or n_keep.dim() != 1 or not n_keep.is_contiguous() or B % n_keep.shape[0]:
            raise ValueError("n_keep must be int32 [seq_mod] with B a multiple of seq_mod")
        seq_mod = n_keep.shape[0]
    if want_out:
        if q is None:
            raise ValueError("q is required for the readout")
        if out is None:
            out = torch.empty(lead + (Hv, Dv), dtype=torch.bfloat16, device=dev)
        elif out.shape != lead + (Hv, Dv) or out.dtype != torch.bfloat16 or not out.is_contiguous():
            raise ValueError("gdr_chunk: out must be contiguous bf16 like v")
    else:
        out = None
    nc = T if num_clean is None else int(num_clean)
    sc = Dk ** -0.5 if scale is None else float(scale)
    lib = _lib.load()
    nbytes = lib.trida_gdr_chunk_workspace_bytes(B, T, Hv)
    ws = workspaces.get(dev, "gdr_chunk", nbytes) if nbytes else None
    rc = lib.trida_gdr_chunk(
        _ptr(q), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), state.data_ptr(), _ptr(out),
        _ptr(state_out), _ptr(n_keep), seq_mod, B, T, Hk, Hv, Dk, Dv, causal_mode, nc, sc, _ptr(ws),
        ws.numel() if ws is not None else 0, _ptr(cu_seqlens), _ptr(state_idx), _stream(dev))
    _lib.check(rc, "trida_gdr_chunk")
    return out


def gdn_snapshot(state: torch.Tensor, snap_state: torch.Tensor, window: Optional[torch.Tensor] = None,
                 snap_window: Optional[torch.Tensor] = None) -> None:
    """Copies recurrent states (fp32) and conv windows (bf16) into snapshot buffers (one launch)."""
    dev = _need_gpu(state, snap_state, window, snap_window)
    _f32(state, "state")
    if snap_state.shape != state.shape or snap_state.dtype != state.dtype:
        raise ValueError("snap_state must match state")
    if not (state.is_contiguous() and snap_state.is_contiguous()):
        raise ValueError("state buffers must be contiguous")
    wn = 0
    if window is not None:
        _bf16(window, "window")
        if snap_window is None or snap_window.shape != window.shape or not window.is_contiguous() \
                or not snap_window.is_contiguous():
            raise ValueError("snap_window must match window (contiguous)")
        wn = window.numel()
    rc = _lib.load().trida_gdn_snapshot(state.data_ptr(), snap_state.data_ptr(), state.numel(), _ptr(window),
                                        _ptr(snap_window), wn, _stream(dev))
    _lib.check(rc, "trida_gdn_snapshot")


def gdn_restore(n_keep: torch.Tensor, *, snap_state: Optional[torch.Tensor] = None,
                state: Optional[torch.Tensor] = None, k: Optional[torch.Tensor] = None,
                v: Optional[torch.Tensor] = None, g: Optional[torch.Tensor] = None,
                beta: Optional[torch.Tensor] = None, snap_window: Optional[torch.Tensor] = None,
                window: Optional[torch.Tensor] = None, preconv: Optional[torch.Tensor] = None,
                skip_full: bool = False, win_idx: Optional[torch.Tensor] = None,
                pre_idx: Optional[torch.Tensor] = None, slots: Optional[int] = None) -> None:
    """Rolls GDN state and/or conv windows back to the accepted prefix n_keep (one launch each).

    The leading dims of every buffer are NB slots (layers stacked on sequences: slot b uses
    n_keep[b % len(n_keep)]). state [NB,Hv,Dv,Dk] fp32, k [NB,T,Hk,Dk], v [NB,T,Hv,Dv] bf16,
    g, beta [NB,T,Hv] fp32, windows [NB,Kc-1,C] bf16, preconv [NB,T,C] bf16 (last dim contiguous).
    Outputs may alias the snapshots. Pool form of the window part: win_idx int32 [NB] picks each slot's
    row of the window pools ([rows, Kc-1, C]), pre_idx int32 [NB] its preconv slot; `slots` is NB then."""
    dev = _need_gpu(n_keep, snap_state, state, k, v, g, beta, snap_window, window, preconv, win_idx, pre_idx)
    if n_keep.dtype != torch.int32 or n_keep.dim() != 1 or not n_keep.is_contiguous():
        raise ValueError("n_keep must be int32 [B]")
    seq_mod = n_keep.shape[0]
    NB = T = Hk = Hv = Dk = Dv = C = Kc = 0
    x_sb = x_st = 0
    if state is not None:
        for t, n in ((snap_state, "snap_state"), (state, "state"), (g, "g"), (beta, "beta")):
            _f32(t, n)
        _bf16(k, "k")
        _bf16(v, "v")
        NB, Hv, Dv, Dk = state.shape
        T, Hk = k.shape[1], k.shape[2]
        if snap_state.shape != state.shape or k.shape != (NB, T, Hk, Dk) or v.shape != (NB, T, Hv, Dv) \
                or g.shape != (NB, T, Hv) or beta.shape != g.shape:
            raise ValueError("restore: state / block row shapes disagree")
        if not all(t.is_contiguous() for t in (snap_state, state, k, v, g, beta)):
            raise ValueError("restore: state and block rows must be contiguous")
    if window is not None:
        _bf16(window, "window")
        _bf16(snap_window, "snap_window")
        _bf16(preconv, "preconv")
        NBw, Km1, C = window.shape
        Kc = Km1 + 1
        if win_idx is not None or pre_idx is not None:
            if slots is None:
                raise ValueError("restore: the pool form (win_idx / pre_idx) needs slots = NB")
            NBw = int(slots)
            _i32(win_idx, "win_idx", NBw)
            _i32(pre_idx, "pre_idx", NBw)
        if NB and NBw != NB:
            raise ValueError("restore: window slots differ from state slots")
        NB = NBw
        T = preconv.shape[1] if not T else T
        if snap_window.shape[1:] != window.shape[1:] or (win_idx is None and snap_window.shape != window.shape) \
                or (win_idx is None and window.shape[0] != NB) or (pre_idx is None and preconv.shape[0] != NB) \
                or preconv.shape[2] != C or preconv.shape[1] != T or preconv.stride(2) != 1:
            raise ValueError("restore: window / preconv shapes disagree")
        _idx_range(win_idx, min(window.shape[0], snap_window.shape[0]), "win_idx")
        _idx_range(pre_idx, preconv.shape[0], "pre_idx")
        x_sb, x_st = preconv.stride(0), preconv.stride(1)
    if NB == 0 or NB % seq_mod:
        raise ValueError("restore: nothing to do or slots not a multiple of len(n_keep)")
    rc = _lib.load().trida_gdn_restore(
        _ptr(snap_state), _ptr(state), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(snap_window), _ptr(window),
        _ptr(preconv), n_keep.data_ptr(), NB, seq_mod, T, Hk, Hv, Dk, Dv, C, Kc, x_sb, x_st, int(skip_full),
        _ptr(win_idx), _ptr(pre_idx), _stream(dev))
    _lib.check(rc, "trida_gdn_restore")


# --------------------------------------------------------------------------------------------------
# attention
MASK_VERIFY, MASK_DRAFT, MASK_CANVAS = 0, 1, 2


def attn_canvas(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, prefix_len: torch.Tensor, *,
                mask_mode: int, n_clean: int = 0, scale: Optional[float] = None,
                gate: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                max_keys: int = 0, splits: int = 0, out_frag: bool = False) -> torch.Tensor:
    """Canvas attention of a block of T rows against a bf16 KV cache (split-K, MFMA).

    q [B, T, Hq, D] bf16 contiguous; k_cache, v_cache [B, Hkv, Lmax, D] bf16 contiguous with the
    block's keys already at [prefix_len, prefix_len + T); prefix_len [B] int32 on the device.
    mask_mode: MASK_VERIFY (causal), MASK_DRAFT (bidirectional block) or MASK_CANVAS (rows < n_clean
    causal). gate (optional) is [B, T, Hq, D]-indexable with a contiguous last dim: the output is
    multiplied by sigmoid(gate). Returns out [B, T, Hq, D] bf16. out_frag: out is instead a buffer for the rows
    [B * T, Hq * D] (B * T <= 48) in the fragment order ws_gemm_frag reads."""
    dev = _need_gpu(q, k_cache, v_cache, prefix_len, gate, out)
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16(t, n)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    B, T, Hq, D = q.shape
    _, Hkv, Lmax, Dk = k_cache.shape
    if k_cache.shape[0] != B or v_cache.shape != k_cache.shape or Dk != D or Hq % Hkv:
        raise ValueError("q / cache shapes disagree")
    if prefix_len.dtype != torch.int32 or prefix_len.shape != (B,) or not prefix_len.is_contiguous():
        raise ValueError("prefix_len must be int32 [B]")
    g_row = g_head = 0
    if gate is not None:
        _bf16(gate, "gate")
        if gate.shape != (B, T, Hq, D) or gate.stride(3) != 1 or gate.stride(0) != T * gate.stride(1):
            raise ValueError("gate must be [B, T, Hq, D] with a contiguous last dim and packed batch rows")
        g_row, g_head = gate.stride(1), gate.stride(2)
    if out_frag:
        if out is None:
            raise ValueError("attn_canvas: out_frag needs an out buffer")
        _frag_buf(out, Hq * D, "out")
    elif out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 tensor shaped like q")
    lib = _lib.load()
    mk = max_keys if max_keys > 0 else Lmax
    scr = workspaces.get(dev, "attn_canvas", lib.trida_attn_canvas_scratch_bytes(B, T, Hq, Hkv, D, mk, splits))
    sc = D ** -0.5 if scale is None else float(scale)
    fn = lib.trida_attn_canvas_frag if out_frag else lib.trida_attn_canvas
    rc = fn(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), prefix_len.data_ptr(), _ptr(gate), g_row, g_head,
            out.data_ptr(), B, T, Hq, Hkv, D, Lmax, mask_mode, n_clean, sc, mk, splits, scr.data_ptr(), scr.numel(),
            _stream(dev))
    _lib.check(rc, "trida_attn_canvas")
    return out


# --------------------------------------------------------------------------------------------------
# weight-streaming GEMM (decode-step projections)
WS_MAX_M = 48
WS_STORE, WS_PARTS, WS_SILU = 0, 1, 2


def ws_shuffle(w: torch.Tensor, *, pair_halves: bool = False, col_scale: Optional[torch.Tensor] = None,
               zero_centred: bool = True) -> torch.Tensor:
    """The weight-streaming layout of a torch Linear weight w [N, K] bf16 (N % 16 == 0, K % 32 == 0): a new
    bf16 tensor of N * K elements (flat). pair_halves: w = [gate; up] (N / 2 rows each), interleaved so
    the SwiGLU epilogue finds each gate row beside its up row. col_scale [K] bf16: an RMSNorm weight folded
    into the columns (bf16(w * (1 + c)) when zero_centred, else bf16(w * c)) for ws_gemm_norm."""
    dev = _need_gpu(w, col_scale)
    _bf16(w, "w")
    N, Kd = w.shape
    if w.stride(1) != 1:
        raise ValueError("ws_shuffle: w needs contiguous rows")
    if col_scale is not None:
        _bf16(col_scale, "col_scale")
        if col_scale.numel() != Kd or not col_scale.is_contiguous():
            raise ValueError("ws_shuffle: col_scale must be K contiguous elements")
    wp = torch.empty(N * Kd, dtype=torch.bfloat16, device=dev)
    rc = _lib.load().trida_wsgemm_shuffle(w.data_ptr(), N, Kd, w.stride(0), int(pair_halves), _ptr(col_scale),
                                          int(zero_centred), wp.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_wsgemm_shuffle")
    return wp


def ws_plan(N: int, Kd: int, epilogue: int) -> int:
    """Partial planes the weight-streaming GEMM writes for (N, K) with `epilogue` (1 unless WS_PARTS)."""
    kg = ctypes.c_int32(0)
    rc = _lib.load().trida_wsgemm_plan(N, Kd, epilogue, ctypes.byref(kg))
    _lib.check(rc, "trida_wsgemm_plan")
    return kg.value


def ws_gemm(x: torch.Tensor, wp: torch.Tensor, N: int, out: torch.Tensor, *, epilogue: int = WS_STORE) -> torch.Tensor:
    """x [M, K] bf16 (M <= 48, contiguous rows) times the weight in ws_shuffle layout (N rows):
    WS_STORE: out [M, N] bf16 = x @ w.T; WS_PARTS: out fp32 [kg, M, N] partial planes (kg = ws_plan);
    WS_SILU: out [M, N / 2] bf16 = silu(x @ gate.T) * (x @ up.T) over a pair_halves weight."""
    dev = _need_gpu(x, wp, out)
    _bf16(x, "x")
    M, Kd = x.shape
    if x.stride(1) != 1 or wp.numel() != N * Kd:
        raise ValueError("ws_gemm: x needs contiguous rows and wp N * K elements")
    if epilogue == WS_PARTS:
        kg = ws_plan(N, Kd, epilogue)
        if out.dtype != torch.float32 or not out.is_contiguous() or out.numel() < kg * M * N:
            raise ValueError(f"ws_gemm: partial planes need a contiguous fp32 out of >= {kg} x {M} x {N}")
        o_st = N
    else:
        width = N // 2 if epilogue == WS_SILU else N
        _bf16(out, "out")
        if out.dim() != 2 or out.shape[0] < M or out.shape[1] < width or out.stride(1) != 1:
            raise ValueError(f"ws_gemm: out must be [>= {M}, >= {width}] bf16 with contiguous rows")
        o_st = out.stride(0)
    rc = _lib.load().trida_wsgemm(x.data_ptr(), x.stride(0), wp.data_ptr(), M, N, Kd, epilogue, out.data_ptr(), o_st,
                                  _stream(dev))
    _lib.check(rc, "trida_wsgemm")
    return out


def ws_argmax_splits(N: int, Kd: int) -> int:
    """Column splits (one per workgroup) of the argmax epilogue of an [N, K] weight-streaming GEMM."""
    S = int(_lib.load().trida_wsgemm_argmax_splits(N, Kd))
    if S <= 0:
        raise ValueError(f"ws_gemm_argmax: shape N={N} K={Kd} not supported")
    return S


def ws_gemm_argmax(x: torch.Tensor, wp: torch.Tensor, N: int, pval: torch.Tensor, pidx: torch.Tensor, *,
                   logits: Optional[torch.Tensor] = None) -> None:
    """The LM head of a greedy verify with its argmax fused in (trida_wsgemm_argmax): x [M, K] bf16 (M <= 48,
    contiguous rows) times the ws_shuffle'd head (N rows); pval fp32 / pidx int32 [M, S] (S =
    ws_argmax_splits(N, K)) receive each row's (bf16 logit max, first column) within each column split;
    logits [M, N] bf16, when given, receives the logits as ws_gemm's store epilogue would."""
    dev = _need_gpu(x, wp, pval, pidx, logits)
    _bf16(x, "x")
    M, Kd = x.shape
    S = ws_argmax_splits(N, Kd)
    if x.stride(1) != 1 or wp.numel() != N * Kd:
        raise ValueError("ws_gemm_argmax: x needs contiguous rows and wp N * K elements")
    if pval.dtype != torch.float32 or pidx.dtype != torch.int32 or not pval.is_contiguous() \
            or not pidx.is_contiguous() or pval.numel() < M * S or pidx.numel() < M * S:
        raise ValueError(f"ws_gemm_argmax: pval fp32 / pidx int32 of >= {M} x {S} contiguous elements")
    o_st = 0
    if logits is not None:
        _bf16(logits, "logits")
        if logits.dim() != 2 or logits.shape[0] < M or logits.shape[1] < N or logits.stride(1) != 1:
            raise ValueError("ws_gemm_argmax: logits must be [>= M, >= N] bf16 with contiguous rows")
        o_st = logits.stride(0)
    rc = _lib.load().trida_wsgemm_argmax(x.data_ptr(), x.stride(0), wp.data_ptr(), M, N, Kd, 0, _ptr(logits), o_st,
                                         pval.data_ptr(), pidx.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_wsgemm_argmax")


def ws_gemm_argmax_conf(x: torch.Tensor, wp: torch.Tensor, N: int, pval: torch.Tensor, pidx: torch.Tensor,
                        psum: torch.Tensor) -> None:
    """ws_gemm_argmax with each split's softmax denominator too (trida_wsgemm_argmax_conf): psum fp32 [M, S]
    receives sum exp(x - pval) over the split's bf16 logits. For argmax_conf_splits (a denoise pass's readout)."""
    dev = _need_gpu(x, wp, pval, pidx, psum)
    _bf16(x, "x")
    M, Kd = x.shape
    S = ws_argmax_splits(N, Kd)
    if x.stride(1) != 1 or wp.numel() != N * Kd:
        raise ValueError("ws_gemm_argmax_conf: x needs contiguous rows and wp N * K elements")
    for t, dt, name in ((pval, torch.float32, "pval"), (pidx, torch.int32, "pidx"), (psum, torch.float32, "psum")):
        if t.dtype != dt or not t.is_contiguous() or t.numel() < M * S:
            raise ValueError(f"ws_gemm_argmax_conf: {name} must be contiguous {dt} of >= {M} x {S} elements")
    rc = _lib.load().trida_wsgemm_argmax_conf(x.data_ptr(), x.stride(0), wp.data_ptr(), M, N, Kd, 0, None, 0,
                                              pval.data_ptr(), pidx.data_ptr(), psum.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_wsgemm_argmax_conf")


CONF_MAX_SPLITS = 256  # column splits argmax_conf_splits reduces (trida_argmax_conf_splits)


def argmax_conf_splits(pval: torch.Tensor, pidx: torch.Tensor, psum: torch.Tensor, *, B: int, R: int, out=None):
    """row_argmax's (argmax, conf) from the per-split triples of ws_gemm_argmax_conf, rows [B, R] (pval / pidx /
    psum [B, R, S]). out: (argmax int64, conf fp32) [B, >= R] with the same row stride and contiguous rows."""
    dev = _need_gpu(pval, pidx, psum)
    n = pval.numel()
    if n % (B * R) or pidx.numel() != n or psum.numel() != n or pval.dtype != torch.float32 \
            or pidx.dtype != torch.int32 or psum.dtype != torch.float32 \
            or not (pval.is_contiguous() and pidx.is_contiguous() and psum.is_contiguous()):
        raise ValueError("argmax_conf_splits: pval / psum fp32 and pidx int32 [B, R, S], contiguous")
    S = n // (B * R)
    if out is None:
        out = (torch.empty((B, R), dtype=torch.int64, device=dev), torch.empty((B, R), dtype=torch.float32, device=dev))
    am, conf = out
    if am.dtype != torch.int64 or conf.dtype != torch.float32 or am.stride() != conf.stride() or am.stride(1) != 1 \
            or am.shape[0] != B or am.shape[1] < R or conf.shape[0] != B or conf.shape[1] < R:
        raise ValueError("argmax_conf_splits: out must be int64 / fp32 [B, >= R] with equal strides")
    rc = _lib.load().trida_argmax_conf_splits(pval.data_ptr(), pidx.data_ptr(), psum.data_ptr(), B, R, S,
                                              am.data_ptr(), conf.data_ptr(), am.stride(0), _stream(dev))
    _lib.check(rc, "trida_argmax_conf_splits")
    return out


def greedy_accept_splits(pval: torch.Tensor, pidx: torch.Tensor, drafts: torch.Tensor, *, R: int,
                         n_live: Optional[torch.Tensor] = None, ctx_len: Optional[torch.Tensor] = None,
                         want_argmax: bool = True, out=None):
    """greedy_accept from the per-split (max, first index) pairs of ws_gemm_argmax: pval / pidx [B, R, S]
    (the GEMM's [M = B R, S] rows), drafts [B, K] int64. Same outputs and semantics as greedy_accept."""
    dev = _need_gpu(pval, pidx, drafts, n_live, ctx_len)
    B = drafts.shape[0]
    if pval.dtype != torch.float32 or pidx.dtype != torch.int32 or pval.numel() % (B * R) \
            or pval.numel() != pidx.numel() or not pval.is_contiguous() or not pidx.is_contiguous():
        raise ValueError("greedy_accept_splits: pval fp32 / pidx int32 [B, R, S], contiguous")
    S = pval.numel() // (B * R)
    if drafts.dtype != torch.int64 or drafts.dim() != 2 or drafts.stride(1) != 1:
        raise ValueError("drafts must be int64 [B, K] with a contiguous last dim")
    K = drafts.shape[1]
    if out is None:
        am = torch.empty((B, R), dtype=torch.int64, device=dev) if want_argmax else None
        out = (am, torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int64, device=dev),
               torch.empty(B, dtype=torch.int64, device=dev))
    am, n_acc, bonus, crop = out
    rc = _lib.load().trida_greedy_accept_splits(
        pval.data_ptr(), pidx.data_ptr(), B, R, S, _ptr(drafts), K, drafts.stride(0), _ptr(n_live), _ptr(ctx_len),
        _ptr(am), n_acc.data_ptr(), bonus.data_ptr(), crop.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_greedy_accept_splits")
    return out


def ss_chunks(dim: int) -> int:
    """Columns of the per-row sums of squares residual_parts writes (256-element chunks)."""
    return int(_lib.load().trida_residual_ss_chunks(dim))


def residual_parts(h: torch.Tensor, parts: Optional[torch.Tensor], n_parts: int, ss: torch.Tensor,
                   h_frag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """h += bf16(sum of the first n_parts planes of parts) in place (bf16 residual stream [rows, dim], planes
    fp32 [>= n_parts, rows, dim] contiguous; n_parts = 0: h unchanged) and ss [rows, ss_chunks(dim)] fp32 = the
    per-chunk sums of h^2 that ws_gemm_norm reads. h_frag: the updated h once more, in the fragment order
    ws_gemm_frag reads (rows <= 48)."""
    dev = _need_gpu(h, parts, ss, h_frag)
    rows, dim = h.shape
    if ss.dtype != torch.float32 or not ss.is_contiguous() or ss.numel() < rows * ss_chunks(dim):
        raise ValueError("residual_parts: ss must be contiguous fp32 [rows, ss_chunks(dim)]")
    if n_parts and (parts is None or parts.dtype != torch.float32 or not parts.is_contiguous()
                    or parts.numel() < n_parts * rows * dim):
        raise ValueError("residual_parts: parts must be contiguous fp32 holding n_parts x rows x dim")
    if h_frag is not None:
        _frag_buf(h_frag, dim, "h_frag")
    rc = _lib.load().trida_residual_parts_frag(h.data_ptr(), h.stride(0), _ptr(parts), n_parts, rows * dim, rows,
                                               dim, ss.data_ptr(), _ptr(h_frag), _stream(dev))
    _lib.check(rc, "trida_residual_parts")
    return h


WS_X_FRAG, WS_OUT_FRAG = 1, 2


def ws_frag_numel(Kd: int) -> int:
    """bf16 elements of the fragment order of a weight-streaming GEMM's X with K = Kd columns (any M <= 48)."""
    n = int(_lib.load().trida_ws_frag_elems(Kd))
    if n <= 0:
        raise ValueError("ws_frag_numel: K must be a positive multiple of 32")
    return n


def ws_frag(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x [M, K] bf16 (M <= 48, contiguous rows) in the fragment order the weight-streaming GEMM reads with
    x_frag (flat bf16, ws_frag_numel(K) elements; rows >= M left unwritten)."""
    dev = _need_gpu(x, out)
    _bf16(x, "x")
    M, Kd = x.shape
    if x.stride(1) != 1:
        raise ValueError("ws_frag: x needs contiguous rows")
    if out is None:
        out = torch.empty(ws_frag_numel(Kd), dtype=torch.bfloat16, device=dev)
    _frag_buf(out, Kd, "out")
    rc = _lib.load().trida_ws_frag(x.data_ptr(), x.stride(0), M, Kd, out.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_ws_frag")
    return out


def _frag_buf(t: torch.Tensor, Kd: int, name: str) -> None:
    _bf16(t, name)
    if not t.is_contiguous() or t.numel() < ws_frag_numel(Kd):
        raise ValueError(f"{name}: a fragment-order buffer needs {ws_frag_numel(Kd)} contiguous bf16 elements")


def ws_gemm_frag(xf: torch.Tensor, M: int, wp: torch.Tensor, N: int, out: torch.Tensor, *,
                 ss: Optional[torch.Tensor] = None, eps: float = 1e-6, epilogue: int = WS_STORE,
                 out_frag: bool = False) -> torch.Tensor:
    """ws_gemm (ss None) or ws_gemm_norm (ss given) of the M rows of X held in fragment order in xf
    (ws_frag, or a producer's fragment-order output; K = wp.numel() // N). out_frag: the bf16 output of
    WS_STORE / WS_SILU goes to out in fragment order (ws_frag_numel of the output width), the next GEMM's X.
    Bitwise the row-major results."""
    dev = _need_gpu(xf, wp, out, ss)
    Kd = wp.numel() // N
    _frag_buf(xf, Kd, "xf")
    if not 1 <= M <= WS_MAX_M:
        raise ValueError(f"ws_gemm_frag: need 1 <= M <= {WS_MAX_M}")
    if ss is not None and (ss.dtype != torch.float32 or not ss.is_contiguous() or ss.numel() < M * ss_chunks(Kd)):
        raise ValueError("ws_gemm_frag: ss must be contiguous fp32 [M, ss_chunks(K)]")
    width = N // 2 if epilogue == WS_SILU else N
    o_st = 0
    if epilogue == WS_PARTS:
        if out_frag:
            raise ValueError("ws_gemm_frag: partial planes have no fragment order")
        kg = ws_plan(N, Kd, epilogue)
        if out.dtype != torch.float32 or not out.is_contiguous() or out.numel() < kg * M * N:
            raise ValueError(f"ws_gemm_frag: partial planes need a contiguous fp32 out of >= {kg} x {M} x {N}")
    elif out_frag:
        _frag_buf(out, width, "out")
    else:
        _bf16(out, "out")
        if out.dim() != 2 or out.shape[0] < M or out.shape[1] < width or out.stride(1) != 1:
            raise ValueError(f"ws_gemm_frag: out must be [>= {M}, >= {width}] bf16 with contiguous rows")
        o_st = out.stride(0)
    flags = WS_X_FRAG | (WS_OUT_FRAG if out_frag else 0)
    rc = _lib.load().trida_wsgemm_ex(xf.data_ptr(), 0, _ptr(ss), eps, wp.data_ptr(), M, N, Kd, epilogue,
                                     out.data_ptr(), o_st, flags, _stream(dev))
    _lib.check(rc, "trida_wsgemm_ex")
    return out


def ws_headnorm_planes(N: int, Kd: int, heads: int) -> int:
    """Partial planes ws_gemm_headnorm writes for an [N, K] weight over `heads` heads of X."""
    kg = ctypes.c_int32(0)
    rc = _lib.load().trida_wsgemm_headnorm_planes(N, Kd, heads, ctypes.byref(kg))
    _lib.check(rc, "trida_wsgemm_headnorm_planes")
    return kg.value


def ws_gemm_headnorm(uf: torch.Tensor, M: int, wp: torch.Tensor, N: int, ss_parts: torch.Tensor, heads: int,
                     out: torch.Tensor, *, eps: float = 1e-6) -> int:
    """Partial planes (fp32 [kg, M, N], kg = ws_headnorm_planes) of the M rows of u in fragment order (uf, from
    gdr_recurrent_gnorm) times the ws_shuffle'd weight, each head's partial sums of a row scaled by
    rsqrt(sum of the row's ss_parts of that head / head width + eps): the out projection of the gated
    RMSNorm's output. Returns kg."""
    dev = _need_gpu(uf, wp, ss_parts, out)
    Kd = wp.numel() // N
    _frag_buf(uf, Kd, "uf")
    kg = ws_headnorm_planes(N, Kd, heads)
    if ss_parts.dtype != torch.float32 or not ss_parts.is_contiguous() or ss_parts.numel() < M * Kd // 8:
        raise ValueError("ws_gemm_headnorm: ss_parts must be contiguous fp32 [M, heads, K / heads / 8]")
    if out.dtype != torch.float32 or not out.is_contiguous() or out.numel() < kg * M * N:
        raise ValueError(f"ws_gemm_headnorm: out must be contiguous fp32 of >= {kg} x {M} x {N}")
    if not 1 <= M <= WS_MAX_M:
        raise ValueError(f"ws_gemm_headnorm: need 1 <= M <= {WS_MAX_M}")
    rc = _lib.load().trida_wsgemm_headnorm(uf.data_ptr(), wp.data_ptr(), M, N, Kd, ss_parts.data_ptr(), heads, eps,
                                           out.data_ptr(), _stream(dev))
    _lib.check(rc, "trida_wsgemm_headnorm")
    return kg


def ws_gemm_norm(h: torch.Tensor, ss: torch.Tensor, wp: torch.Tensor, N: int, out: torch.Tensor, *,
                 eps: float = 1e-6, epilogue: int = WS_STORE) -> torch.Tensor:
    """ws_gemm of rmsnorm(h) against a weight shuffled with the norm weight as col_scale: h the raw bf16
    residual stream [M, K] (M <= 48), ss its per-chunk sums of squares from residual_parts; row m is scaled
    by rsqrt(mean(h_m^2) + eps) in the epilogue. Epilogue WS_STORE or WS_SILU."""
    dev = _need_gpu(h, ss, wp, out)
    _bf16(h, "h")
    M, Kd = h.shape
    if h.stride(1) != 1 or wp.numel() != N * Kd:
        raise ValueError("ws_gemm_norm: h needs contiguous rows and wp N * K elements")
    if ss.dtype != torch.float32 or not ss.is_contiguous() or ss.numel() < M * ss_chunks(Kd):
        raise ValueError("ws_gemm_norm: ss must be contiguous fp32 [M, ss_chunks(K)]")
    width = N // 2 if epilogue == WS_SILU else N
    _bf16(out, "out")
    if out.dim() != 2 or out.shape[0] < M or out.shape[1] < width or out.stride(1) != 1:
        raise ValueError(f"ws_gemm_norm: out must be [>= {M}, >= {width}] bf16 with contiguous rows")
    rc = _lib.load().trida_wsgemm_norm(h.data_ptr(), h.stride(0), ss.data_ptr(), eps, wp.data_ptr(), M, N, Kd,
                                       epilogue, out.data_ptr(), out.stride(0), _stream(dev))
    _lib.check(rc, "trida_wsgemm_norm")
    return out


# --------------------------------------------------------------------------------------------------
# row-wise decoder kernels
def add_rmsnorm(x: torch.Tensor, r: Optional[torch.Tensor], w: torch.Tensor, out: torch.Tensor, *,
                eps: float = 1e-6, zero_centred: bool = True) -> torch.Tensor:
    """x += r (in place, bf16 residual stream; r may be None), out = rmsnorm(x) * (1 + w) (or * w).
    x, r, out: [rows, dim] bf16 with contiguous rows; w [dim] bf16."""
    dev = _need_gpu(x, r, w, out)
    rows, dim = x.shape
    rc = _lib.load().trida_add_rmsnorm(x.data_ptr(), _ptr(r), w.data_ptr(), out.data_ptr(), rows, dim, x.stride(0),
                                       r.stride(0) if r is not None else 0, out.stride(0), eps, int(zero_centred),
                                       _stream(dev))
    _lib.check(rc, "trida_add_rmsnorm")
    return out


def add_rmsnorm_parts(x: torch.Tensor, parts: torch.Tensor, n_parts: int, w: torch.Tensor, out: torch.Tensor, *,
                      eps: float = 1e-6, zero_centred: bool = True) -> torch.Tensor:
    """add_rmsnorm whose residual is the sum of the first n_parts planes of parts (fp32 [>= n_parts, rows, dim],
    contiguous: the WS_PARTS output of ws_gemm), summed in plane order and rounded to bf16."""
    dev = _need_gpu(x, parts, w, out)
    rows, dim = x.shape
    if parts.dtype != torch.float32 or not parts.is_contiguous() or parts.numel() < n_parts * rows * dim:
        raise ValueError("add_rmsnorm_parts: parts must be contiguous fp32 holding n_parts x rows x dim")
    rc = _lib.load().trida_add_rmsnorm_parts(x.data_ptr(), parts.data_ptr(), n_parts, rows * dim, w.data_ptr(),
                                             out.data_ptr(), rows, dim, x.stride(0), out.stride(0), eps,
                                             int(zero_centred), _stream(dev))
    _lib.check(rc, "trida_add_rmsnorm_parts")
    return out


def silu_mul(gu: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = silu(gu[:, :I]) * gu[:, I:] for gu [rows, 2I] bf16."""
    dev = _need_gpu(gu, out)
    rows, two_i = gu.shape
    rc = _lib.load().trida_silu_mul(gu.data_ptr(), out.data_ptr(), rows, two_i // 2, gu.stride(0), out.stride(0),
                                    _stream(dev))
    _lib.check(rc, "trida_silu_mul")
    return out


def gated_rmsnorm(o: torch.Tensor, z: torch.Tensor, w: torch.Tensor, out: torch.Tensor, *, eps: float = 1e-6,
                  out_frag: bool = False):
    """Per value head: out = bf16(rmsnorm(o)) * w * silu(z). o, out [rows, H, Dv] contiguous bf16;
    z [rows, >= H*Dv] bf16 with contiguous rows; w [Dv] bf16. out_frag: out is instead a buffer for the
    rows [rows, H * Dv] in the fragment order ws_gemm_frag reads (rows <= 48)."""
    dev = _need_gpu(o, z, w, out)
    rows, H, Dv = o.shape
    if out_frag:
        _frag_buf(out, H * Dv, "out")
        fn = _lib.load().trida_gated_rmsnorm_frag
    else:
        fn = _lib.load().trida_gated_rmsnorm
    rc = fn(o.data_ptr(), z.data_ptr(), w.data_ptr(), out.data_ptr(), rows, H, Dv, z.stride(0), eps, _stream(dev))
    _lib.check(rc, "trida_gated_rmsnorm")
    return out


def attn_prep(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, pos0: torch.Tensor,
              slot0: torch.Tensor, q_out: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *,
              Hq: int, Hkv: int, D: int, rot_dim: int, rope_theta: float, eps: float = 1e-6) -> None:
    """Per-head q/k RMSNorm + partial RoPE; q to q_out [B, T, Hq, D], k / v into the caches
    [B, Hkv, Lmax, D] at slots slot0[b] + t. qkv [B, T, >= (2Hq + 2Hkv) D] bf16 with packed rows."""
    dev = _need_gpu(qkv, q_norm_w, k_norm_w, pos0, slot0, q_out, k_cache, v_cache)
    B, T = qkv.shape[0], qkv.shape[1]
    if qkv.stride(0) != T * qkv.stride(1) or qkv.stride(2) != 1:
        raise ValueError("qkv rows must be packed")
    rc = _lib.load().trida_attn_prep(qkv.data_ptr(), qkv.stride(1), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
                                     pos0.data_ptr(), slot0.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(),
                                     v_cache.data_ptr(), B, T, Hq, Hkv, D, k_cache.shape[2], rot_dim, rope_theta,
                                     eps, _stream(dev))
    _lib.check(rc, "trida_attn_prep")
