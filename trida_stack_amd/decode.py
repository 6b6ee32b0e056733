"""Decoders on MI355X: autoregressive baseline and self-speculative decoding.

Mirrors inference/zoro-1/mlx/trida_mlx/decode.py (SamplingParams, DecodeStats, ar_generate,
selfspec_generate; decode.py:35-387) over the GPU runtime of trida_stack_amd.model:

  selfspec_generate(..., n, denoise_steps=0)   the reference canvas algorithm (bd_bidir_shift):
      cold start [t0, MASK x (2n-2)]; verify round [pending, spec_1..spec_{n-1}, MASK x (n-1)] with
      n_clean = n; spec_i verified against row i; all accepted -> clean = row n-1, new specs = rows
      n..2n-2; reject at i -> emit the accepted specs + correction, next step cold.
  selfspec_generate(..., n, denoise_steps=D)   draft-then-verify over a block of n: D block-diffusion
      passes over [t0, MASK x n] (each unmasks the most confident MASK slots, shift readout), then a
      token-causal verify pass over [t0, d_1..d_n], greedy acceptance and rollback of the hybrid state
      (KV crop + GDN restore to 1 + n_acc rows).

Acceptance runs in the fused gfx950 kernels (greedy: split-V argmax + wave prefix scan; temperature > 0:
speculative rejection sampling, trida_stack_amd.sampling); the host syncs once per step to emit tokens. Greedy decoding is lossless w.r.t. ar_generate up to bf16
numerics (the verify rows are the AR computation).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Iterator, List, Optional

import torch

from . import kernels as K
from .model import SeqCache, TridaRuntime


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_k: int = 50
    top_p: float = 0.95
    seed: Optional[int] = None

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0


@dataclass
class DecodeStats:
    mode: str = ""
    prompt_tokens: int = 0
    reused_tokens: int = 0
    new_tokens: int = 0
    forwards: int = 0
    cold_forwards: int = 0
    steps: int = 0
    accept_hist: list = field(default_factory=list)
    prefill_s: float = 0.0
    decode_s: float = 0.0
    finish_reason: str = "length"
    stop_token: Optional[int] = None

    @property
    def tokens_per_forward(self) -> float:
        return self.new_tokens / self.forwards if self.forwards else 0.0

    @property
    def decode_tps(self) -> float:
        return self.new_tokens / self.decode_s if self.decode_s else 0.0

    def as_dict(self) -> dict:
        return {"mode": self.mode, "prompt_tokens": self.prompt_tokens, "reused_tokens": self.reused_tokens,
                "new_tokens": self.new_tokens, "forwards": self.forwards, "cold_forwards": self.cold_forwards,
                "steps": self.steps, "tokens_per_forward": round(self.tokens_per_forward, 3),
                "accept_hist": self.accept_hist, "prefill_s": round(self.prefill_s, 4),
                "decode_s": round(self.decode_s, 4), "decode_tok_s": round(self.decode_tps, 2),
                "finish_reason": self.finish_reason}


class _Emitter:
    """Applies max_new_tokens / EOS to emitted chunks and records stats (decode.py:228-257)."""

    def __init__(self, stats: DecodeStats, max_new: int, eos: set):
        self.stats, self.max_new, self.eos, self.done = stats, max_new, eos, False

    def __call__(self, toks: list) -> list:
        out = []
        for t in toks:
            if t in self.eos:
                self.done = True
                self.stats.finish_reason = "stop"
                self.stats.stop_token = t
                break
            out.append(t)
            if self.stats.new_tokens + len(out) >= self.max_new:
                self.done = True
                self.stats.finish_reason = "length"
                break
        self.stats.new_tokens += len(out)
        return out


def _argmax1(logits: torch.Tensor) -> int:
    am, _ = K.row_argmax(logits.reshape(1, -1), want_conf=False)
    return int(am[0])


def _prefill(rt: TridaRuntime, cache: SeqCache, prompt: list, stats: DecodeStats) -> torch.Tensor:
    t = time.perf_counter()
    todo = prompt[len(cache.tokens[0]):]
    stats.prompt_tokens, stats.reused_tokens = len(prompt), len(cache.tokens[0])
    if not todo:
        raise ValueError("prompt fully cached; callers must leave at least one token to prefill")
    logits = rt.prefill(cache, todo)
    torch.cuda.synchronize(rt.dev)
    stats.prefill_s = time.perf_counter() - t
    return logits


# ----------------------------------------------------------------------------- AR
def ar_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                sp: SamplingParams, stats: Optional[DecodeStats] = None) -> Iterator[list]:
    """Causal decoding (decode.py:273-293): greedy, or sampled through trida_stack_amd.sampling."""
    stats = stats or DecodeStats()
    if not sp.greedy:
        from .sampling import ar_sample_generate

        yield from ar_sample_generate(rt, cache, prompt, max_new_tokens=max_new_tokens, eos_ids=eos_ids, sp=sp,
                                      stats=stats)
        return
    stats.mode = "causal"
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t = time.perf_counter()
    while True:
        tok = _argmax1(logits)
        out = emit([tok])
        if out:
            yield out
        if emit.done:
            break
        logits = rt.ar_step(cache, tok)
        stats.forwards += 1
    stats.decode_s = time.perf_counter() - t


# ----------------------------------------------------------------------------- pure block diffusion
def diffusion_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                       mask_id: int, canvas: int = 32, threshold: float = 0.9, max_steps: Optional[int] = None,
                       stats: Optional[DecodeStats] = None) -> Iterator[list]:
    """Greedy block diffusion with the LowConfidenceShift commit gate (qwen3_5_diffusion.py:449-632,
    1180-1270). A block [seed, MASK x (canvas - 1)] is denoised by draft passes (prefix plus the whole
    block visible; MASK rows read the block-end GDN state): position i takes the prediction of the
    logits of position i - 1 when its softmax confidence exceeds `threshold`, or, when no masked
    position passes, only the most confident one does (first on ties); rounds repeat until no mask is
    left or `max_steps` (default: canvas) ran. A causal forward then commits the block; the whole
    block is emitted and the argmax of its last logit seeds the next one."""
    stats = stats or DecodeStats()
    stats.mode = "diffusion"
    CL = int(canvas)
    if CL < 2:
        raise ValueError("canvas must hold the seed and at least one masked position")
    max_steps = CL if max_steps is None else int(max_steps)
    seed = _argmax1(_prefill(rt, cache, prompt, stats))
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    dev = rt.dev
    ids = torch.full((1, CL), mask_id, dtype=torch.int64, device=dev)
    neg = torch.tensor(float("-inf"), device=dev)
    t = time.perf_counter()
    while True:
        ids.fill_(mask_id)
        ids[0, 0] = seed
        for _ in range(max_steps):
            logits = rt.draft(cache, ids)[0]
            stats.forwards += 1
            pred, conf = K.row_argmax(logits[: CL - 1])  # row i - 1 predicts position i
            cur = ids[0, 1:]
            masked = cur == mask_id
            score = torch.where(masked, conf, neg)
            take = score > threshold
            if not bool(take.any()):
                best = int(torch.nonzero(score == score.max())[0])  # first most confident masked position
                take[best] = True
            ids[0, 1:] = torch.where(take, pred, cur)
            if not bool((ids[0, 1:] == mask_id).any()):
                break
        block = ids[0].tolist()
        logits = rt.prefill(cache, block)  # the causal commit forward (state and KV persisted)
        stats.forwards += 1
        stats.steps += 1
        out = emit(block)
        if out:
            yield out
        if emit.done:
            break
        seed = _argmax1(logits)
    stats.decode_s = time.perf_counter() - t


# ----------------------------------------------------------------------------- self-spec
def selfspec_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                      sp: SamplingParams, mask_id: int, n: int = 4, stats: Optional[DecodeStats] = None,
                      denoise_steps: int = 0) -> Iterator[list]:
    """Self-speculative decoding (decode.py:297-387); see the module docstring for the two variants.
    Sampling parameters with temperature > 0 run the rejection-sampling versions of both variants
    (trida_stack_amd.sampling)."""
    if not sp.greedy:
        from . import sampling as S

        stats = stats or DecodeStats()
        if denoise_steps > 0:
            yield from S.blockspec_sample_generate(rt, cache, prompt, max_new_tokens=max_new_tokens, eos_ids=eos_ids,
                                                   sp=sp, mask_id=mask_id, block=n, denoise=denoise_steps,
                                                   stats=stats)
        else:
            yield from S.selfspec_sample_generate(rt, cache, prompt, max_new_tokens=max_new_tokens, eos_ids=eos_ids,
                                                  sp=sp, mask_id=mask_id, n=n, stats=stats)
        return
    if denoise_steps > 0:
        yield from _blockspec(rt, cache, prompt, max_new_tokens=max_new_tokens, eos_ids=eos_ids, mask_id=mask_id,
                              block=n, denoise=denoise_steps, stats=stats)
        return
    stats = stats or DecodeStats()
    stats.mode = f"self-spec(N={n})"
    stats.accept_hist = [0] * n
    blk, Kd = 2 * n - 1, n - 1
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t_start = time.perf_counter()
    t0 = _argmax1(logits)
    t0_emitted = False
    pending = specs = None
    dev = rt.dev
    while not emit.done:
        if specs is not None:  # ---- verify round
            L = rt.canvas(cache, [pending] + specs + [mask_id] * (n - 1), n, as_float=False)
            stats.forwards += 1
            drafts = torch.as_tensor([specs], dtype=torch.int64, device=dev)
            am, n_acc, _, _ = K.greedy_accept(L[None], drafts)
            vals = am[0].tolist()
            acc = int(n_acc[0])
            if acc < Kd:  # rejected at spec `acc`: emit accepted specs + correction, next step cold
                rt.commit(cache, 1 + acc)
                stats.accept_hist[acc] += 1
                out = emit(specs[:acc] + [vals[acc]])
                t0, t0_emitted = vals[acc], True
                pending = specs = None
            else:  # all accepted: n tokens this forward
                rt.commit(cache, n)
                stats.accept_hist[Kd] += 1
                out = emit(specs + [vals[n - 1]])
                pending, specs = vals[n - 1], vals[n:blk]
        else:  # ---- cold start
            L = rt.canvas(cache, [t0] + [mask_id] * (blk - 1), n, rows=n if rt.skip_rows else None, as_float=False)
            stats.forwards += 1
            stats.cold_forwards += 1
            am, _ = K.row_argmax(L[:n], want_conf=False)
            vals = am.tolist()
            rt.commit(cache, 1)
            out = emit(([] if t0_emitted else [t0]) + [vals[0]])
            t0_emitted = True
            pending, specs = vals[0], vals[1:n]
        if out:
            yield out
    stats.decode_s = time.perf_counter() - t_start


class BlockSpecStep:
    """One batched draft-then-verify step on device buffers of fixed shape (so a whole step can be
    replayed from a HIP graph): denoise passes, verify, greedy acceptance, rollback.

    Inputs: t0 [B] int64 (the pending token, already emitted). Outputs after run(): canvas [B, block+1]
    (row 0 = t0, rows 1.. = drafts), n_acc [B] int32, bonus [B] int64 (next t0)."""

    def __init__(self, rt: TridaRuntime, cache: SeqCache, block: int, denoise: int):
        self.rt, self.cache, self.block, self.denoise = rt, cache, block, denoise
        B = cache.B
        dev = rt.dev
        self.per = [block // denoise + (1 if p < block % denoise else 0) for p in range(denoise)]
        self.t0 = torch.zeros(B, dtype=torch.int64, device=dev)
        self.canvas = torch.full((B, block + 1), rt.mask_id, dtype=torch.int64, device=dev)
        self.masked = torch.ones(B, block, dtype=torch.bool, device=dev)
        self.ctx = torch.zeros(B, dtype=torch.int64, device=dev)
        self.n_keep = torch.zeros(B, dtype=torch.int32, device=dev)
        self.am = torch.empty(B, block + 1, dtype=torch.int64, device=dev)
        self.n_acc = torch.empty(B, dtype=torch.int32, device=dev)
        self.bonus = torch.empty(B, dtype=torch.int64, device=dev)
        self.crop = torch.empty(B, dtype=torch.int64, device=dev)
        self.d_am = torch.empty(B, block + 1, dtype=torch.int64, device=dev)
        self.d_conf = torch.empty(B, block + 1, dtype=torch.float32, device=dev)

    def run(self) -> None:
        rt, cache, blk = self.rt, self.cache, self.block
        self.canvas.fill_(rt.mask_id)
        self.canvas[:, 0] = self.t0
        self.masked.fill_(True)
        for p in range(self.denoise):
            L = rt.forward(self.canvas, cache, "draft")
            # row j predicts slot j + 1 (shift readout); the last row is not used
            with K.timed("row_argmax"):
                K.row_argmax(L, out=(self.d_am, self.d_conf))
            # the per[p] most confident MASK slots (ties: the lower slot first) take their predictions
            K.unmask_top(self.d_am, self.d_conf, self.masked, self.canvas, self.per[p])
        vt = K.timed("verify_step").__enter__()
        L = rt.forward(self.canvas, cache, "verify")
        self.ctx.copy_(cache.length)
        with K.timed("greedy_accept"):
            K.greedy_accept(L, self.canvas[:, 1:], ctx_len=self.ctx, out=(self.am, self.n_acc, self.bonus, self.crop))
        torch.add(self.n_acc, 1, out=self.n_keep)
        cache.pending = {"T": blk + 1}
        rt.commit(cache, self.n_keep)
        vt.__exit__(None, None, None)
        self.t0.copy_(self.bonus)

    # ---------------------------------------------------------------- HIP-graph replay
    graph = None

    def capture(self) -> None:
        """Records one whole step (every kernel of the denoise and verify forwards, the acceptance and the
        rollback) into a HIP graph; replay() then launches it with one call. The step reads lengths and
        positions on the device, so one graph serves every step; the attention key splits are planned for
        the cache capacity (splits past a sequence's keys exit at once). The warm-up runs that precede the
        capture are undone (cache state, lengths and t0 restored), so the cache is left as it was."""
        rt, cache = self.rt, self.cache
        cache.ctx_hint = max(cache.ctx_hint, cache.Lmax)
        snap, t0 = cache.snapshot(), self.t0.clone()
        side = torch.cuda.Stream(rt.dev)
        side.wait_stream(torch.cuda.current_stream(rt.dev))
        with torch.cuda.stream(side):
            for _ in range(2):  # workspaces, allocator pools and library handles exist before capture
                self.run()
                cache.restore(snap)
                self.t0.copy_(t0)
        torch.cuda.current_stream(rt.dev).wait_stream(side)
        torch.cuda.synchronize(rt.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run()
        torch.cuda.synchronize(rt.dev)
        self.graph = g

    def replay(self) -> None:
        """One step from the captured graph (capture() first)."""
        self.graph.replay()


def _blockspec(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
               mask_id: int, block: int, denoise: int, stats: Optional[DecodeStats],
               graph: bool = True) -> Iterator[list]:
    stats = stats or DecodeStats()
    stats.mode = f"self-spec(block={block}, denoise={denoise})"
    stats.accept_hist = [0] * (block + 1)
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t_start = time.perf_counter()
    step = BlockSpecStep(rt, cache, block, denoise)
    t0 = _argmax1(logits)
    out = emit([t0])
    if out:
        yield out
    step.t0.fill_(t0)
    use_graph = graph and rt.dev.type == "cuda"
    while not emit.done:
        if use_graph and step.graph is None and stats.steps >= 1:
            step.capture()
        if step.graph is not None:
            step.replay()
        else:
            step.run()
        stats.forwards += denoise + 1
        stats.steps += 1
        packed = torch.cat([step.canvas[0, 1:], step.bonus[:1], step.n_acc[:1].to(torch.int64)]).tolist()
        acc = packed[-1]
        cache.tokens[0].extend([t0] + packed[:acc])  # the committed rows: pending token + accepted drafts
        cache.ctx_hint = len(cache.tokens[0])
        stats.accept_hist[acc] += 1
        chunk = packed[:acc] + [packed[block]]
        t0 = packed[block]
        out = emit(chunk)
        if out:
            yield out
    stats.decode_s = time.perf_counter() - t_start
