"""Sampled decoding on MI355X: temperature / top-k / top-p sampling for the AR baseline and speculative
rejection sampling for self-spec (the canvas algorithm and the batched draft-then-verify step).

Mirrors the sampled branches of inference/zoro-1/mlx/trida_mlx/decode.py:
  ar_generate         tok ~ truncated_probs(logits)                                   (decode.py:283)
  selfspec_generate   verify round: ratio p(d)/q(d), accept while ratio >= 1 or u < ratio, correction
                      from norm(max(0, P - q)), clean + new specs drawn from P[n-1:blk], new q = P[n:blk];
                      cold start: clean + specs drawn from P[:n], q = P[1:n]        (decode.py:333-387)
  truncated_probs     temperature, top-k, top-p                                    (decode.py:102-130)
and the role of the vLLM plugin's sampled self-spec step (_ss_sample_verify, _ss_draft_gumbel_kernel:
inference/zoro-1/vllm/vllm_native_diffusion/qwen3_5_diffusion.py:250-285, 787-880), whose q rows are
full-vocabulary fp32 distributions kept per draft slot (qwen3_5_diffusion.py:779).

Token draws. The reference draws with an RNG (mx.random.categorical / Gumbel noise) that has no
uniform -> token contract. Here every draw is the inverse CDF in vocabulary order at one seeded uniform,
token = min{x : cdf(x) > u * mass}, computed on the GPU by the sampled-acceptance kernels (a verify
with no drafts draws from P_0; the draft passes draw from row statistics computed once, trida_sample_rows). The MASK id is banned from every sampled row, drafts and verify alike
(qwen3_5_diffusion.py:820), so the AR baseline and self-spec share one target distribution.
"""
from __future__ import annotations

import time
from typing import Iterator, List, Optional

import torch

from . import kernels as K
from .model import SeqCache, TridaRuntime


class Sampler:
    """Seeded sampling of truncated distributions on the device (one generator per decode)."""

    def __init__(self, sp, device: torch.device, ban_id: int = -1):
        from .decode import LogitRules

        if sp.temperature <= 0:
            raise ValueError("Sampler needs temperature > 0 (temperature 0 is greedy decoding)")
        if sp.top_k > K.MAX_TOP_K:
            raise ValueError(f"top_k <= {K.MAX_TOP_K} is supported (got {sp.top_k})")
        self.T, self.top_k, self.top_p = float(sp.temperature), int(max(sp.top_k, 0)), float(sp.top_p)
        self.ban = int(ban_id)
        self.dev = torch.device(device)
        self.gen = torch.Generator(device=self.dev)
        if sp.seed is None:
            self.gen.seed()
        else:
            self.gen.manual_seed(int(sp.seed))
        self.bad = torch.zeros(1, dtype=torch.int32, device=self.dev)  # any nonzero kernel status so far
        # sp.banned / sp.gate (apply_ban, decode.py:76-99), applied once to each fp32 row buffer by prepare()
        self.rules = LogitRules(sp, self.dev)

    def prepare(self, lf: torch.Tensor, raw_p: Optional[torch.Tensor] = None) -> torch.Tensor:
        """fp32 logit rows [..., V] with the ban / gate rules applied in place (before any statistics)."""
        return self.rules.apply(lf, raw_p) if self.rules.active else lf

    def uniform(self, *shape) -> torch.Tensor:
        return torch.rand(shape, generator=self.gen, device=self.dev, dtype=torch.float32)

    def _note(self, status: torch.Tensor) -> None:
        self.bad |= (status != 0).any().to(torch.int32)

    def check(self) -> None:
        """Raises when any sampled row so far had a NaN / +inf logit or no finite logit."""
        if int(self.bad):
            raise FloatingPointError("sampled decoding met a NaN / +inf logit or a row with no finite logit")

    def draw(self, logits: torch.Tensor, u: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One token per row of logits [..., V] (bf16 or fp32, already prepared) from the truncated
        distribution."""
        V = logits.shape[-1]
        x = logits.reshape(-1, V)
        if x.dtype != torch.float32 or x.stride(1) != 1:
            x = x.float().contiguous()
        n = x.shape[0]
        u = self.uniform(n) if u is None else u
        none = torch.empty((n, 0), dtype=torch.int64, device=self.dev)
        _, tok, _, _, st = K.sample_accept(x.view(n, 1, V), None, none, None, u, temperature=self.T,
                                           top_k=self.top_k, top_p=self.top_p, ban_id=self.ban)
        self._note(st)
        return tok.view(logits.shape[:-1])

    def draw_given(self, lf: torch.Tensor, stats, u: torch.Tensor) -> torch.Tensor:
        """One token per row of fp32 logits [B, R, V] from their truncated distributions, given the
        statistics of `stats` (no second truncation pass)."""
        return K.sample_rows(lf, stats, u, temperature=self.T, ban_id=self.ban)

    def stats(self, lf: torch.Tensor):
        m, thr, zk, st = K.truncate_stats(lf, temperature=self.T, top_k=self.top_k, top_p=self.top_p,
                                          ban_id=self.ban)
        self._note(st)
        return m, thr, zk

    def probs(self, lf: torch.Tensor, stats=None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Truncated distributions P [B, R, V] fp32 of fp32 logits [B, R, V]."""
        stats = self.stats(lf) if stats is None else stats
        return K.truncated_probs(lf, stats, temperature=self.T, ban_id=self.ban, out=out)

    def accept(self, pf: torch.Tensor, q: torch.Tensor, drafts: torch.Tensor, *, ctx_len=None, n_live=None,
               u_accept: Optional[torch.Tensor] = None, u_sample: Optional[torch.Tensor] = None, out=None):
        """Rejection-sampling acceptance of a verify pass (fp32 logits [B, R, V], q [B, K, V])."""
        B, Kd = drafts.shape
        ua = self.uniform(B, Kd) if u_accept is None else u_accept
        us = self.uniform(B) if u_sample is None else u_sample
        res = K.sample_accept(pf, q, drafts, ua, us, temperature=self.T, top_k=self.top_k, top_p=self.top_p,
                              ban_id=self.ban, ctx_len=ctx_len, n_live=n_live, out=out)
        self._note(res[4])
        return res


# ----------------------------------------------------------------------------- AR (sampled)
def ar_sample_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                       sp, stats) -> Iterator[list]:
    """Sampled causal decoding (decode.py:273-293, the sampled branch at :283)."""
    from .decode import _Emitter, _prefill, _room

    stats.mode = "causal"
    smp = Sampler(sp, rt.dev, ban_id=rt.mask_id)
    raw = smp.rules.raw_buffer(1, rt.dev)
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t = time.perf_counter()
    while True:
        row = smp.prepare(logits.reshape(1, -1), raw)
        tok = int(smp.draw(row)[0])
        smp.check()
        if raw is not None:
            smp.rules.note(raw.tolist())
        out = emit([tok])
        if out:
            yield out
        if emit.done:
            break
        _room(cache, 1)
        logits = rt.ar_step(cache, tok)
        stats.forwards += 1
    stats.decode_s = time.perf_counter() - t


# ----------------------------------------------------------------------------- self-spec (sampled)
def selfspec_sample_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int,
                             eos_ids: set, sp, mask_id: int, n: int, stats) -> Iterator[list]:
    """Sampled self-spec with the bd_bidir_shift canvas (decode.py:297-387, sampled branches): one
    host read per forward (acceptance, correction or clean token, and the next specs together)."""
    from .decode import _Emitter, _prefill, _room

    stats.mode = f"self-spec(N={n})"
    stats.accept_hist = [0] * n
    smp = Sampler(sp, rt.dev, ban_id=mask_id)
    blk, Kd = 2 * n - 1, n - 1
    raw = smp.rules.raw_buffer(blk, rt.dev)
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t_start = time.perf_counter()
    t0 = int(smp.draw(smp.prepare(logits.reshape(1, -1), None if raw is None else raw[:1]))[0])
    if raw is not None:
        smp.rules.note(raw[:1].tolist())
    t0_emitted = False
    pending = specs = spec_q = None
    dev = rt.dev
    while not emit.done:
        _room(cache, blk)
        if specs is not None:  # ---- verify round
            L = rt.canvas(cache, [pending] + specs + [mask_id] * (n - 1), n, as_float=False)
            stats.forwards += 1
            pf = smp.prepare(L.float()[None], raw)                     # [1, blk, V]
            drafts = torch.as_tensor([specs], dtype=torch.int64, device=dev)
            n_acc, tok, _, _, _ = smp.accept(pf, spec_q, drafts)
            new = smp.draw(pf[0, n:blk])                                # next specs (used when all accepted)
            vals = torch.cat([n_acc.to(torch.int64), tok, new]).tolist()
            smp.check()
            acc, tk, new_specs = vals[0], vals[1], vals[2:]
            if raw is not None:  # rows that saw real context (decode.py:358)
                smp.rules.note(raw[: acc + 1 if acc < Kd else n].tolist())
            if acc < Kd:  # rejected at spec `acc`: tk is the correction, next step cold
                rt.commit(cache, 1 + acc)
                stats.accept_hist[acc] += 1
                out = emit(specs[:acc] + [tk])
                t0, t0_emitted = tk, True
                pending = specs = spec_q = None
            else:  # all accepted: tk is the clean token drawn from P[n-1]
                rt.commit(cache, n)
                stats.accept_hist[Kd] += 1
                out = emit(specs + [tk])
                pending, specs = tk, new_specs
                spec_q = smp.probs(pf[:, n:blk].contiguous())
        else:  # ---- cold start
            L = rt.canvas(cache, [t0] + [mask_id] * (blk - 1), n, rows=n if rt.skip_rows else None, as_float=False)
            stats.forwards += 1
            stats.cold_forwards += 1
            pf = smp.prepare(L[:n].float()[None], None if raw is None else raw[:n])  # [1, n, V]
            if raw is not None:
                smp.rules.note(raw[:1].tolist())
            vals = smp.draw(pf[0]).tolist()
            smp.check()
            spec_q = smp.probs(pf[:, 1:n].contiguous())
            rt.commit(cache, 1)
            out = emit(([] if t0_emitted else [t0]) + [vals[0]])
            t0_emitted = True
            pending, specs = vals[0], vals[1:n]
        if out:
            yield out
    stats.decode_s = time.perf_counter() - t_start


class SampledBlockSpecStep:
    """One batched draft-then-verify step with speculative rejection sampling, on device buffers of fixed
    shape: `denoise` block-diffusion passes over [t0, MASK x block], a token-causal verify pass,
    rejection-sampling acceptance (the correction, or the bonus when every draft is accepted, becomes
    the next t0) and the hybrid rollback to 1 + n_acc rows per sequence (ragged KV crops and GDN
    restores).

    The passes unmask the block in ascending slot order: pass p draws the `per[p]` lowest still-masked
    slots, each from the truncated distribution of its row of that pass's logits (shift readout: row s
    predicts slot s), and keeps that distribution as the slot's q row. Which slots a pass unmasks is
    fixed before anything is drawn, and a slot's q depends only on lower slots' drafts, so every draft
    is distributed exactly as its q given the drafts before it: the condition under which speculative
    rejection sampling reproduces the verify distribution (decode.py:333-354; the reference's canvas
    algorithm draws its specs from rows that see only lower positions, decode.py:361-378).

    Inputs: t0 [B] int64. Outputs after run(): canvas [B, block+1] (row 0 = t0, rows 1.. = drafts),
    n_acc [B] int32, token [B] int64 (next t0). q rows: [B, block, V] fp32 (the reference layout,
    qwen3_5_diffusion.py:779). trace: a list to which run() appends the pass inputs (for parity tests),
    or None."""

    def __init__(self, rt: TridaRuntime, cache: SeqCache, block: int, denoise: int, sampler: Sampler):
        if not 1 <= denoise <= block:
            raise ValueError(f"need 1 <= denoise ({denoise}) <= block ({block})")
        self.rt, self.cache, self.block, self.denoise, self.smp = rt, cache, block, denoise, sampler
        B, V = cache.B, rt.cfg.vocab
        dev = rt.dev
        self.per = [block // denoise + (1 if p < block % denoise else 0) for p in range(denoise)]
        self.start = [sum(self.per[:p]) for p in range(denoise)]
        # per pass: the logits rows [B, per] it reads (0..per-1 of the pass's LM-head rows) and the q rows
        # [B, per] it writes (its slots)
        self.sel = [torch.arange(k, device=dev).repeat(B, 1).contiguous() for k in self.per]
        self.slots = [torch.arange(s, s + k, device=dev).repeat(B, 1).contiguous()
                      for s, k in zip(self.start, self.per)]
        self.t0 = torch.zeros(B, dtype=torch.int64, device=dev)
        self.canvas = torch.full((B, block + 1), rt.mask_id, dtype=torch.int64, device=dev)
        self.ctx = torch.zeros(B, dtype=torch.int64, device=dev)
        self.n_keep = torch.zeros(B, dtype=torch.int32, device=dev)
        self.out = (torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int64, device=dev),
                    torch.empty(B, dtype=torch.int64, device=dev), None, torch.empty(B, dtype=torch.int32, device=dev))
        self.lf = torch.empty(B * max(self.per) * V, dtype=torch.float32, device=dev)  # a pass's rows, fp32
        self.q = torch.zeros(B, block, V, dtype=torch.float32, device=dev)             # q row per draft slot
        self.pf = torch.empty(B, block + 1, V, dtype=torch.float32, device=dev)        # verify rows
        self.ua = torch.zeros(B, block, dtype=torch.float32, device=dev)               # acceptance uniforms
        self.us = torch.zeros(B, dtype=torch.float32, device=dev)                      # correction / bonus
        # raw gate probabilities of the verify rows, when the decode keeps gate notes
        self.raw_p = None
        if sampler.rules.log is not None:
            self.raw_p = torch.zeros(B, block + 1, sampler.rules.n_gate, dtype=torch.float32, device=dev)
        self.trace: Optional[list] = None

    @property
    def n_acc(self) -> torch.Tensor:
        return self.out[0]

    @property
    def token(self) -> torch.Tensor:
        return self.out[1]

    def run(self) -> None:
        self.draft()
        self.draw_uniforms()
        self.verify()

    def draw_uniforms(self) -> None:
        """The acceptance uniforms of the verify pass (drawn before it, so the verify half has no RNG)."""
        B = self.cache.B
        self.ua.copy_(self.smp.uniform(B, self.block))
        self.us.copy_(self.smp.uniform(B))

    def draft(self) -> None:
        """The denoising passes: canvas = [t0, drafts], q rows of the drafted slots."""
        rt, cache, smp = self.rt, self.cache, self.smp
        B, V = cache.B, rt.cfg.vocab
        self.canvas.fill_(rt.mask_id)
        self.canvas[:, 0] = self.t0
        for p in range(self.denoise):
            k, s0 = self.per[p], self.start[p]
            # the LM head only for the rows of the slots this pass unmasks
            L = rt.forward(self.canvas, cache, "draft", rows=k, row0=s0)
            lf = self.lf[: B * k * V].view(B, k, V)
            with K.timed("draft_sample"):
                K.gather_rows(L, self.sel[p], out=lf)                     # widen to fp32
                smp.prepare(lf)
                st = smp.stats(lf)
                u = smp.uniform(B * k)
                x = smp.draw_given(lf, st, u)                            # [B, k]
            if self.trace is not None:
                self.trace.append({"lf": lf.clone(), "u": u.clone(), "x": x.clone(), "start": s0})
            self.canvas[:, 1 + s0: 1 + s0 + k] = x
            with K.timed("draft_q"):  # q[slot] = P of the slot's row, written in place
                K.truncated_probs_rows(lf, st, self.sel[p], self.slots[p], self.q, temperature=smp.T, ban_id=smp.ban)

    def verify(self) -> None:
        """The verify pass, rejection-sampling acceptance with the drawn uniforms, and the rollback; t0 = the
        correction or bonus token."""
        rt, cache, blk, smp = self.rt, self.cache, self.block, self.smp
        vt = K.timed("verify_step").__enter__()
        rt.forward(self.canvas, cache, "verify", logits_out=self.pf)  # fp32 logits from the LM head
        smp.prepare(self.pf, self.raw_p)
        self.ctx.copy_(cache.length)
        ua, us = self.ua, self.us
        with K.timed("sample_accept"):
            smp.accept(self.pf, self.q, self.canvas[:, 1:], ctx_len=self.ctx, u_accept=ua, u_sample=us, out=self.out)
        if self.trace is not None:
            self.trace.append({"pf": self.pf.clone(), "q": self.q.clone(), "drafts": self.canvas[:, 1:].clone(),
                               "ua": ua.clone(), "us": us.clone()})
        torch.add(self.n_acc, 1, out=self.n_keep)
        cache.pending = {"T": blk + 1}
        rt.commit(cache, self.n_keep)
        vt.__exit__(None, None, None)
        self.t0.copy_(self.token)


def blockspec_sample_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int,
                              eos_ids: set, sp, mask_id: int, block: int, denoise: int, stats) -> Iterator[list]:
    """Sampled draft-then-verify decode of one sequence over SampledBlockSpecStep."""
    from .decode import _Emitter, _prefill, _room

    stats.mode = f"self-spec(block={block}, denoise={denoise})"
    stats.accept_hist = [0] * (block + 1)
    smp = Sampler(sp, rt.dev, ban_id=mask_id)
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t_start = time.perf_counter()
    step = SampledBlockSpecStep(rt, cache, block, denoise, smp)
    raw = smp.rules.raw_buffer(1, rt.dev)
    t0 = int(smp.draw(smp.prepare(logits.reshape(1, -1), raw))[0])
    if raw is not None:
        smp.rules.note(raw.tolist())
    out = emit([t0])
    if out:
        yield out
    step.t0.fill_(t0)
    while not emit.done:
        _room(cache, block + 1)
        step.run()
        stats.forwards += denoise + 1
        stats.steps += 1
        packed = torch.cat([step.canvas[0, 1:], step.token[:1], step.n_acc[:1].to(torch.int64)]).tolist()
        smp.check()
        acc = packed[-1]
        if step.raw_p is not None:
            smp.rules.note(step.raw_p[0, : acc + 1].tolist())
        cache.tokens[0].extend([t0] + packed[:acc])
        cache.ctx_hint = len(cache.tokens[0])
        stats.accept_hist[acc] += 1
        t0 = packed[block]
        out = emit(packed[:acc] + [t0])
        if out:
            yield out
    stats.decode_s = time.perf_counter() - t_start


def prefill_batch(rt: TridaRuntime, cache: SeqCache, prompts: List[List[int]]) -> torch.Tensor:
    """Per-sequence causal prefill of ragged prompts into a batched cache. Returns the fp32 last-token
    logits [B, V]."""
    assert len(prompts) == cache.B
    rows = [rt.prefill(cache, p, seq=b) for b, p in enumerate(prompts)]
    cache.ctx_hint = max(len(p) for p in prompts)
    return torch.stack(rows)
