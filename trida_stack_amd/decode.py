"""Decoders on MI355X: autoregressive baseline and self-speculative decoding.

Mirrors inference/zoro-1/mlx/trida_mlx/decode.py (SamplingParams, DecodeStats, ar_generate,
selfspec_generate; decode.py:35-387) over the GPU runtime of trida_stack_amd.model:

  selfspec_generate(..., n, denoise_steps=0)   the reference canvas algorithm (bd_bidir_shift):
      cold start [t0, MASK x (2n-2)]; verify round [pending, spec_1..spec_{n-1}, MASK x (n-1)] with
      n_clean = n; spec_i verified against row i; all accepted -> clean = row n-1, new specs = rows
      n..2n-2; reject at i -> emit the accepted specs + correction, next step cold. Greedy steps run
      as CanvasSpecStep (the next-canvas decision on the device), replayed from one HIP graph.
  selfspec_generate(..., n, denoise_steps=D)   draft-then-verify over a block of n: D block-diffusion
      passes over [t0, MASK x n] (each unmasks the most confident MASK slots, shift readout), then a
      token-causal verify pass over [t0, d_1..d_n], greedy acceptance and rollback of the hybrid state
      (KV crop + GDN restore to 1 + n_acc rows).

Acceptance runs in the fused gfx950 kernels (greedy: split-V argmax + wave prefix scan; temperature > 0:
speculative rejection sampling, trida_stack_amd.sampling); the host syncs once per step to emit tokens. Greedy decoding is lossless w.r.t. ar_generate up to bf16
numerics (the verify rows are the AR computation).
"""
from __future__ import annotations

import collections
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
    # token ids that are never produced (greedy and sampled rows, drafts and verify alike)
    banned: tuple = ()
    # ((token id, min raw probability), ...): the token is allowed only where its probability under the
    # raw logits (temperature 1, no top-k / top-p, after the ban) is at least that value
    gate: tuple = ()
    # when a list: (raw probability, gate) of every exact causal row where a gated token was blocked
    # although the model gave it >= GATE_NOTE_MIN
    gate_log: Optional[list] = None

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0


GATE_NOTE_MIN = 0.05


class LogitRules:
    """SamplingParams.banned / gate in device form for one decode: apply() runs apply_ban
    (inference/zoro-1/mlx/trida_mlx/decode.py:76-99) in place on logit rows (trida_ban_tokens, then
    trida_gate_tokens), and note() records near-miss gate blocks of exact causal rows into
    sp.gate_log (_gate_note, decode.py:63-73). Inactive rules cost nothing."""

    def __init__(self, sp: SamplingParams, device: torch.device):
        dev = torch.device(device)
        ban = sorted({int(i) for i in (sp.banned or ())})
        self.ban = torch.tensor(ban, dtype=torch.int64, device=dev) if ban else None
        gates = [(int(t), float(th)) for t, th in (sp.gate or ())]
        self.gates = gates
        self.gate_ids = torch.tensor([g[0] for g in gates], dtype=torch.int64, device=dev) if gates else None
        self.gate_thr = torch.tensor([g[1] for g in gates], dtype=torch.float32, device=dev) if gates else None
        self.log = sp.gate_log if gates else None

    @property
    def active(self) -> bool:
        return self.ban is not None or self.gate_ids is not None

    @property
    def n_gate(self) -> int:
        return len(self.gates)

    def apply(self, logits: torch.Tensor, raw_p: Optional[torch.Tensor] = None) -> torch.Tensor:
        """logits [..., V] (fp32 or bf16, evenly strided rows) with the rules applied, in place; raw_p
        [rows, n_gate] fp32 receives the gated tokens' raw probabilities: under the softmax of the raw row,
        before the ban, as _gate_note takes them (decode.py:63-73). The gate itself decides on the banned
        row, as apply_ban does (decode.py:88-98)."""
        if raw_p is not None and self.gate_ids is not None:
            K.gate_tokens(logits, self.gate_ids, None, raw_p)  # note-only pass over the raw rows
        if self.ban is not None:
            K.ban_tokens(logits, self.ban)
        if self.gate_ids is not None:
            K.gate_tokens(logits, self.gate_ids, self.gate_thr)
        return logits

    def raw_buffer(self, rows: int, device) -> Optional[torch.Tensor]:
        """A raw-probability buffer for `rows` rows when gate notes are wanted, else None."""
        if self.log is None:
            return None
        return torch.zeros(rows, self.n_gate, dtype=torch.float32, device=device)

    def note(self, raw_rows) -> None:
        """raw_rows: host lists of per-gate raw probabilities of exact causal rows."""
        if self.log is None:
            return
        for row in raw_rows:
            for (tid, thr), p in zip(self.gates, row):
                if thr > 0 and GATE_NOTE_MIN <= p < thr:
                    self.log.append((round(float(p), 4), thr))


def apply_ban(x: torch.Tensor, sp: SamplingParams) -> torch.Tensor:
    """x [..., V] on the GPU with sp.banned at -inf and sp.gate applied, in place (apply_ban,
    decode.py:76-99; greedy and sampled alike, drafts and verify alike)."""
    r = LogitRules(sp, x.device)
    return r.apply(x) if r.active else x


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
    gate_blocked: list = field(default_factory=list)  # raw probabilities of blocked gated tokens (>= 0.05)
    loop_stopped_thinking: bool = False  # the loop guard closed the thinking and the model answered after it
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
                "finish_reason": self.finish_reason,
                **({"gate_blocked": self.gate_blocked} if self.gate_blocked else {}),
                **({"loop_stopped_thinking": True} if self.loop_stopped_thinking else {})}


# ----------------------------------------------------------------------------- loop guard
# Thresholds of the reference's loop guard (decode.py:172-217): a block repeated LOOP_MIN_REPEATS times
# back to back spanning >= LOOP_MIN_SPAN tokens, or a LOOP_WINDOW-token window in which at least
# LOOP_REPEAT_FRAC of the positions end a LOOP_NGRAM-token phrase seen before in the window.
LOOP_MIN_REPEATS = 6
LOOP_MIN_SPAN = 96
LOOP_MAX_PERIOD = 256
LOOP_NGRAM = 16
LOOP_WINDOW = 1536
LOOP_REPEAT_FRAC = 0.5


def _z_array(r: list) -> list:
    """z[i] = length of the longest common prefix of r and r[i:] (z[0] = len(r)); linear time
    (Gusfield's Z algorithm)."""
    m = len(r)
    z = [0] * m
    if m:
        z[0] = m
    lo = hi = 0  # [lo, hi) is the rightmost window known to match a prefix of r
    for i in range(1, m):
        k = min(hi - i, z[i - lo]) if i < hi else 0
        while i + k < m and r[k] == r[i + k]:
            k += 1
        z[i] = k
        if i + k > hi:
            lo, hi = i, i + k
    return z


def looping(hist: list) -> int:
    """The period p of a block that ends `hist` repeated LOOP_MIN_REPEATS times back to back (the tail of
    max(p * LOOP_MIN_REPEATS, LOOP_MIN_SPAN) tokens equals itself shifted by p), for the smallest such
    p <= LOOP_MAX_PERIOD; 0 when there is none (the rule of decode.py:178-195).

    Read backwards from the last token, the tail has period p over `span` tokens exactly when the
    reversed history agrees with itself shifted by p for span - p tokens, i.e. z[p] >= span - p for the
    Z-array of the reversed tail: one linear pass answers every p at once."""
    n = len(hist)
    top = min(LOOP_MAX_PERIOD, n // LOOP_MIN_REPEATS)
    if top < 1 or max(LOOP_MIN_REPEATS, LOOP_MIN_SPAN) > n:
        return 0
    reach = min(n, max(top * LOOP_MIN_REPEATS, LOOP_MIN_SPAN))  # the longest span any p can need
    z = _z_array(hist[: n - reach - 1: -1] if reach < n else hist[::-1])
    for p in range(1, top + 1):
        span = max(p * LOOP_MIN_REPEATS, LOOP_MIN_SPAN)
        if span > n:
            break
        if z[p] >= span - p:
            return p
    return 0


class NgramLoop:
    """Sliding-window repeat detector (decode.py:198-225): over the last `window` positions, the count
    of positions whose `n`-token phrase had already occurred among the `window` phrases before it.

    The window is a ring of (phrase, was-a-repeat) records overwritten in place, with a multiset of
    the phrases it holds; each add is O(n) for the phrase key and O(1) otherwise."""

    def __init__(self, n: int = LOOP_NGRAM, window: int = LOOP_WINDOW, frac: float = LOOP_REPEAT_FRAC):
        self.n, self.window, self.frac = n, window, frac
        self._held = collections.Counter()        # phrase -> occurrences inside the ring
        self._ring: list = [None] * window         # (phrase, repeat flag) records, oldest at _head when full
        self._head = 0
        self._filled = 0
        self._repeats = 0                          # repeat flags set inside the ring
        self._need = frac * window

    def add(self, hist: list) -> bool:
        """Feeds the history after one new token; True once the window is full and mostly repeats."""
        if len(hist) < self.n:
            return False
        phrase = tuple(hist[len(hist) - self.n:])
        repeat = self._held[phrase] > 0            # judged against the window before this position
        if self._filled == self.window:            # the record at _head leaves the window
            old, old_rep = self._ring[self._head]
            self._repeats -= old_rep
            self._held[old] -= 1
            if not self._held[old]:
                del self._held[old]
        else:
            self._filled += 1
        self._ring[self._head] = (phrase, repeat)
        self._head = (self._head + 1) % self.window
        self._held[phrase] += 1
        self._repeats += repeat
        return self._filled == self.window and self._repeats >= self._need


class _Emitter:
    """The stop rules of a decode (decode.py:228-257) applied to each chunk of new tokens: a token of
    `eos` ends it before that token ("stop"), the max_new budget ends it after the token that fills it
    ("length"), and the optional loop guard after the token that completes a loop ("repetition").
    Records new_tokens / finish_reason / stop_token in `stats`. The guard is off unless the class
    attribute is set (the server's --loop-guard)."""

    loop_guard = False

    def __init__(self, stats: DecodeStats, max_new: int, eos: set):
        self.stats, self.max_new, self.eos, self.done = stats, max_new, eos, False
        self.hist: list = []
        self.ngram = NgramLoop()

    def _loops(self) -> bool:
        periodic = len(self.hist) % 8 == 0 and looping(self.hist) > 0
        return periodic or self.ngram.add(self.hist)

    def __call__(self, toks: list) -> list:
        toks = list(toks)
        # where the chunk ends before the guard: at the first EOS, or once the budget is spent (the
        # budget always admits one more token, as a decode step always emits at least one)
        eos_at = next((i for i, t in enumerate(toks) if t in self.eos), len(toks))
        budget = max(1, self.max_new - self.stats.new_tokens)
        limit, reason = eos_at, None
        if budget <= eos_at:
            limit, reason = budget, "length"
        elif eos_at < len(toks):
            reason = "stop"
        out = toks[:limit]
        if self.loop_guard:
            # the guard inspects each token that is kept, except the one that spends the budget
            guarded = limit - 1 if reason == "length" else limit
            for i in range(guarded):
                self.hist.append(out[i])
                if self._loops():
                    out, reason = out[: i + 1], "repetition"
                    break
            else:
                self.hist.extend(out[guarded:])
        else:
            self.hist.extend(out)
        if reason is not None:
            self.done = True
            self.stats.finish_reason = reason
            if reason == "stop":
                self.stats.stop_token = toks[eos_at]
        self.stats.new_tokens += len(out)
        return out


def _room(cache: SeqCache, T: int) -> None:
    """A forward of T rows must fit every sequence's KV cache (the kernels take the committed lengths
    from the device and would write past the capacity)."""
    need = max(len(t) for t in cache.tokens) + T
    if need > cache.Lmax:
        raise ValueError(f"KV cache capacity {cache.Lmax} exceeded ({need} positions needed)")


def _argmax1(logits: torch.Tensor) -> int:
    am, _ = K.row_argmax(logits.reshape(1, -1), want_conf=False)
    return int(am[0])


def _prefill(rt: TridaRuntime, cache: SeqCache, prompt: list, stats: DecodeStats) -> torch.Tensor:
    t = time.perf_counter()
    held = cache.tokens[0]
    if prompt[: len(held)] != held:
        raise ValueError("the cache holds tokens that are not a prefix of the prompt")
    todo = prompt[len(held):]
    stats.prompt_tokens, stats.reused_tokens = len(prompt), len(held)
    if not todo:
        raise ValueError("prompt fully cached; callers must leave at least one token to prefill")
    _room(cache, len(todo))
    logits = rt.prefill(cache, todo)
    torch.cuda.synchronize(rt.dev)
    stats.prefill_s = time.perf_counter() - t
    return logits


def _greedy_row(rules: LogitRules, logits: torch.Tensor, note: bool = True) -> int:
    """The argmax of one exact causal row after the ban / gate rules (which also note gate blocks)."""
    if rules.active:
        raw = rules.raw_buffer(1, logits.device) if note else None
        rules.apply(logits.reshape(1, -1), raw)
        if raw is not None:
            rules.note(raw.tolist())
    return _argmax1(logits)


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
    rules = LogitRules(sp, rt.dev)
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t = time.perf_counter()
    while True:
        tok = _greedy_row(rules, logits)
        out = emit([tok])
        if out:
            yield out
        if emit.done:
            break
        _room(cache, 1)
        logits = rt.ar_step(cache, tok)
        stats.forwards += 1
    stats.decode_s = time.perf_counter() - t


# ----------------------------------------------------------------------------- pure block diffusion
def diffusion_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                       mask_id: int, canvas: int = 32, threshold: float = 0.9, max_steps: Optional[int] = None,
                       stats: Optional[DecodeStats] = None, sp: Optional[SamplingParams] = None) -> Iterator[list]:
    """Greedy block diffusion with the LowConfidenceShift commit gate (qwen3_5_diffusion.py:449-632,
    1180-1270). A block [seed, MASK x (canvas - 1)] is denoised by draft passes (prefix plus the whole
    block visible; MASK rows read the block-end GDN state): position i takes the prediction of the
    logits of position i - 1 when its softmax confidence exceeds `threshold`, or, when no masked
    position passes, only the most confident one does (first on ties); rounds repeat until no mask is
    left or `max_steps` (default: canvas) ran. A causal forward then commits the block; the whole
    block is emitted and the argmax of its last logit seeds the next one. sp.banned / sp.gate apply to
    every row read."""
    stats = stats or DecodeStats()
    stats.mode = "diffusion"
    rules = LogitRules(sp or SamplingParams(temperature=0.0), rt.dev)
    CL = int(canvas)
    if CL < 2:
        raise ValueError("canvas must hold the seed and at least one masked position")
    max_steps = CL if max_steps is None else int(max_steps)
    seed = _greedy_row(rules, _prefill(rt, cache, prompt, stats))
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    dev = rt.dev
    ids = torch.full((1, CL), mask_id, dtype=torch.int64, device=dev)
    neg = torch.tensor(float("-inf"), device=dev)
    t = time.perf_counter()
    while True:
        _room(cache, CL)
        ids.fill_(mask_id)
        ids[0, 0] = seed
        for _ in range(max_steps):
            logits = rt.draft(cache, ids)[0]
            stats.forwards += 1
            rows = logits[: CL - 1]  # row i - 1 predicts position i
            if rules.active:
                rules.apply(rows)
            pred, conf = K.row_argmax(rows)
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
        seed = _greedy_row(rules, logits)
    stats.decode_s = time.perf_counter() - t


# ----------------------------------------------------------------------------- self-spec
def selfspec_generate(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                      sp: SamplingParams, mask_id: int, n: int = 4, stats: Optional[DecodeStats] = None,
                      denoise_steps: int = 0) -> Iterator[list]:
    """Self-speculative decoding (decode.py:297-387); see the module docstring for the two variants.
    Sampling parameters with temperature > 0 run the rejection-sampling versions of both variants
    (trida_stack_amd.sampling). sp.banned / sp.gate apply to every row read (drafts and verify)."""
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
                              block=n, denoise=denoise_steps, stats=stats, sp=sp)
        return
    yield from _canvas_spec(rt, cache, prompt, max_new_tokens=max_new_tokens, eos_ids=eos_ids, sp=sp, mask_id=mask_id,
                            n=n, stats=stats)


def _capture_step(step, cache, state: list) -> "torch.cuda.CUDAGraph":
    """Records step.run() into a HIP graph. Two warm-up runs on a side stream first create workspaces,
    allocator pools and library handles; they are undone (cache state, lengths and the `state` tensors
    restored), so the cache is left as it was. Attention key splits are planned for the cache capacity
    (splits past a sequence's keys exit at once), so one graph serves every step."""
    rt = step.rt
    cache.ctx_hint = max(cache.ctx_hint, cache.Lmax)
    snap = cache.snapshot()
    saved = [t.clone() for t in state]

    def undo():
        cache.restore(snap)
        for t, v in zip(state, saved):
            t.copy_(v)

    side = torch.cuda.Stream(rt.dev)
    side.wait_stream(torch.cuda.current_stream(rt.dev))
    with torch.cuda.stream(side):
        for _ in range(2):
            step.run()
            undo()
    torch.cuda.current_stream(rt.dev).wait_stream(side)
    torch.cuda.synchronize(rt.dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step.run()
    torch.cuda.synchronize(rt.dev)
    undo()
    return g


class CanvasSpecStep:
    """One batched bd_bidir_shift canvas step (decode.py:318-384) on device buffers of fixed shape, so that a
    whole step replays from one HIP graph: the canvas forward (rows < n token-causal; MASK rows see the
    block and read the block-end GDN state), greedy acceptance of the specs against rows 0..n-2, the
    device-side decision of what is emitted and what the next canvas is (trida_canvas_advance), and the
    rollback to the committed rows (KV crop + GDN restore).

    State: canvas [B, 2n-1] ([t0, MASK...] cold, or [pending, specs, MASK...]) and verify [B] (uint8).
    Outputs after run(): emit [B, n] / n_emit [B] (tokens emitted), committed [B, n] / n_keep [B] (rows
    committed), kind [B] (1 for a verify round). rules: the decode's ban / gate rules (every row), or None;
    with gate notes wanted, raw_p [B, 2n-1, n_gate] holds the rows' raw gate probabilities."""

    def __init__(self, rt: TridaRuntime, cache: SeqCache, n: int, rules: Optional[LogitRules] = None):
        if n < 2:
            raise ValueError("the canvas needs n >= 2 (one pending token and at least one spec)")
        self.rt, self.cache, self.n = rt, cache, n
        self.rules = rules if rules is not None and rules.active else None
        B, blk = cache.B, 2 * n - 1
        dev = rt.dev
        i32, i64 = dict(dtype=torch.int32, device=dev), dict(dtype=torch.int64, device=dev)
        self.canvas = torch.full((B, blk), rt.mask_id, **i64)
        self.verify = torch.zeros(B, dtype=torch.uint8, device=dev)
        self.live = torch.zeros(B, **i32)
        self.am = torch.empty(B, blk, **i64)
        self.acc = (torch.empty(B, **i32), torch.empty(B, **i64), torch.empty(B, **i64))
        self.n_keep, self.n_emit, self.kind = torch.zeros(B, **i32), torch.zeros(B, **i32), torch.zeros(B, **i32)
        self.emit, self.committed = torch.zeros(B, n, **i64), torch.zeros(B, n, **i64)
        self.raw_p = None
        if self.rules is not None and self.rules.log is not None:
            self.raw_p = torch.zeros(B, blk, self.rules.n_gate, dtype=torch.float32, device=dev)
        self.graph = None

    def start(self, t0: torch.Tensor) -> None:
        """Cold canvases [t0, MASK...] for every sequence (t0 [B] int64, already emitted)."""
        self.canvas.fill_(self.rt.mask_id)
        self.canvas[:, 0] = t0
        self.verify.zero_()

    def run(self) -> None:
        rt, cache, n = self.rt, self.cache, self.n
        self.live.copy_(self.verify)
        self.live.mul_(n - 1)  # specs that count: n - 1 on a verify canvas, none on a cold one
        n_acc, bonus, crop = self.acc
        if self.rules is None and rt.greedy_head_ok(cache.B * (2 * n - 1)):
            # every canvas row's argmax straight from the LM head's epilogue (no logits written or read)
            pv, pi = rt.forward(self.canvas, cache, "canvas", n_clean=n, head="argmax")
            with K.timed("greedy_accept"):
                K.greedy_accept_splits(pv, pi, self.canvas[:, 1:n], R=2 * n - 1, n_live=self.live,
                                       out=(self.am, n_acc, bonus, crop))
        else:
            L = rt.forward(self.canvas, cache, "canvas", n_clean=n)
            if self.rules is not None:
                self.rules.apply(L, self.raw_p)
            with K.timed("greedy_accept"):
                K.greedy_accept(L, self.canvas[:, 1:n], n_live=self.live, out=(self.am, n_acc, bonus, crop))
        K.canvas_advance(self.am, n_acc, self.canvas, self.verify,
                         (self.n_keep, self.emit, self.n_emit, self.committed, self.kind), rt.mask_id)
        cache.pending = {"T": 2 * n - 1}
        rt.commit(cache, self.n_keep)

    def capture(self) -> None:
        self.graph = _capture_step(self, self.cache, [self.canvas, self.verify])

    def replay(self) -> None:
        self.graph.replay()


def _canvas_spec(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
                 sp: SamplingParams, mask_id: int, n: int, stats: Optional[DecodeStats],
                 graph: bool = True) -> Iterator[list]:
    """Greedy self-spec with the bd_bidir_shift canvas (decode.py:297-387), each step a CanvasSpecStep
    replayed from one HIP graph; the host reads the step's emitted and committed tokens once."""
    stats = stats or DecodeStats()
    stats.mode = f"self-spec(N={n})"
    stats.accept_hist = [0] * n
    rules = LogitRules(sp, rt.dev)
    if mask_id != rt.mask_id:
        raise ValueError(f"mask_id {mask_id} is not the runtime's ({rt.mask_id})")
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t_start = time.perf_counter()
    t0 = _greedy_row(rules, logits)
    out = emit([t0])
    if out:
        yield out
    step = CanvasSpecStep(rt, cache, n, rules)
    step.start(torch.full((1,), t0, dtype=torch.int64, device=rt.dev))
    use_graph = graph and rt.dev.type == "cuda"
    while not emit.done:
        _room(cache, 2 * n - 1)
        if use_graph and step.graph is None and stats.forwards >= 1:
            step.capture()
        if step.graph is not None:
            step.replay()
        else:
            step.run()
        stats.forwards += 1
        stats.steps += 1
        packed = torch.cat([step.kind[:1].to(torch.int64), step.n_emit[:1].to(torch.int64),
                            step.n_keep[:1].to(torch.int64), step.emit[0], step.committed[0]]).tolist()
        kind, ne, nk = packed[0], packed[1], packed[2]
        toks, committed = packed[3: 3 + ne], packed[3 + n: 3 + n + nk]
        cache.tokens[0].extend(committed)
        cache.ctx_hint = len(cache.tokens[0])
        if kind:
            stats.accept_hist[ne - 1] += 1
        else:
            stats.cold_forwards += 1
        if step.raw_p is not None:  # rows that saw real context (decode.py:358)
            rules.note(step.raw_p[0, :ne].tolist())
        out = emit(toks)
        if out:
            yield out
    stats.decode_s = time.perf_counter() - t_start


class BlockSpecStep:
    """One batched draft-then-verify step on device buffers of fixed shape (so a whole step can be
    replayed from a HIP graph): denoise passes, verify, greedy acceptance, rollback.

    Inputs: t0 [B] int64 (the pending token, already emitted). Outputs after run(): canvas [B, block+1]
    (row 0 = t0, rows 1.. = drafts), n_acc [B] int32, bonus [B] int64 (next t0). rules: the ban / gate
    rules of the decode (applied to every draft and verify row), or None; with gate notes wanted,
    raw_p [B, block+1, n_gate] holds the verify rows' raw gate probabilities."""

    def __init__(self, rt: TridaRuntime, cache: SeqCache, block: int, denoise: int,
                 rules: Optional[LogitRules] = None):
        self.rt, self.cache, self.block, self.denoise = rt, cache, block, denoise
        self.rules = rules if rules is not None and rules.active else None
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
        self.raw_p = None
        if self.rules is not None and self.rules.log is not None:
            self.raw_p = torch.zeros(B, block + 1, self.rules.n_gate, dtype=torch.float32, device=dev)

    def run(self) -> None:
        self.draft()
        self.verify()

    def draft(self) -> None:
        """The denoising passes: canvas = [t0, drafts]."""
        rt, cache = self.rt, self.cache
        self.canvas.fill_(rt.mask_id)
        self.canvas[:, 0] = self.t0
        self.masked.fill_(True)
        B, blk = cache.B, self.block
        # without ban / gate rules (which edit the logits) the LM head reduces its rows to per-split (max,
        # index, softmax denominator) triples itself: no logits are written or read back
        fused = self.rules is None and rt.greedy_head_ok(B * blk) and rt.argmax_conf_ok()
        for p in range(self.denoise):
            # row j predicts slot j + 1 (shift readout); the last row is not used
            if fused:
                pv, pi, ps = rt.forward(self.canvas, cache, "draft", rows=blk, head="argmax_conf")
                with K.timed("row_argmax"):
                    K.argmax_conf_splits(pv, pi, ps, B=B, R=blk, out=(self.d_am, self.d_conf))
            else:
                L = rt.forward(self.canvas, cache, "draft")
                if self.rules is not None:
                    self.rules.apply(L)
                with K.timed("row_argmax"):
                    K.row_argmax(L, out=(self.d_am, self.d_conf))
            # the per[p] most confident MASK slots (ties: the lower slot first) take their predictions
            K.unmask_top(self.d_am, self.d_conf, self.masked, self.canvas, self.per[p])

    def verify(self) -> None:
        """The verify pass over the canvas, greedy acceptance and the rollback; t0 = the bonus token."""
        rt, cache, blk = self.rt, self.cache, self.block
        vt = K.timed("verify_step").__enter__()
        if self.rules is None and rt.greedy_head_ok(cache.B * (blk + 1)):
            # the LM head leaves per-split (max, index) pairs, not logits: acceptance reads 67 KB, not 16 MB
            pv, pi = rt.forward(self.canvas, cache, "verify", head="argmax")
            self.ctx.copy_(cache.length)
            with K.timed("greedy_accept"):
                K.greedy_accept_splits(pv, pi, self.canvas[:, 1:], R=blk + 1, ctx_len=self.ctx,
                                       out=(self.am, self.n_acc, self.bonus, self.crop))
        else:
            L = rt.forward(self.canvas, cache, "verify")
            if self.rules is not None:
                self.rules.apply(L, self.raw_p)
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
        rollback) into a HIP graph; replay() then launches it with one call (_capture_step)."""
        self.graph = _capture_step(self, self.cache, [self.t0])

    def replay(self) -> None:
        """One step from the captured graph (capture() first)."""
        self.graph.replay()


def _blockspec(rt: TridaRuntime, cache: SeqCache, prompt: list, *, max_new_tokens: int, eos_ids: set,
               mask_id: int, block: int, denoise: int, stats: Optional[DecodeStats],
               sp: Optional[SamplingParams] = None, graph: bool = True) -> Iterator[list]:
    stats = stats or DecodeStats()
    stats.mode = f"self-spec(block={block}, denoise={denoise})"
    stats.accept_hist = [0] * (block + 1)
    rules = LogitRules(sp or SamplingParams(temperature=0.0), rt.dev)
    logits = _prefill(rt, cache, prompt, stats)
    emit = _Emitter(stats, max_new_tokens, eos_ids)
    t_start = time.perf_counter()
    step = BlockSpecStep(rt, cache, block, denoise, rules)
    t0 = _greedy_row(rules, logits)
    out = emit([t0])
    if out:
        yield out
    step.t0.fill_(t0)
    use_graph = graph and rt.dev.type == "cuda"
    while not emit.done:
        _room(cache, block + 1)
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
        if step.raw_p is not None:
            rules.note(step.raw_p[0, : acc + 1].tolist())
        cache.tokens[0].extend([t0] + packed[:acc])  # the committed rows: pending token + accepted drafts
        cache.ctx_hint = len(cache.tokens[0])
        stats.accept_hist[acc] += 1
        chunk = packed[:acc] + [packed[block]]
        t0 = packed[block]
        out = emit(chunk)
        if out:
            yield out
    stats.decode_s = time.perf_counter() - t_start
