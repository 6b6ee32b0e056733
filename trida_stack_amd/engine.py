"""Mode-switching generation engine (the drop-in surface of inference/zoro-1/mlx/trida_mlx/engine.py:54-271):
``Engine(model, mode="self-spec", gen_block=N, prefill_chunk=512, prompt_cache=True, fused_gdn=...,
cache_slots=3).generate_ids(prompt, max_tokens=..., sampling=..., mode=..., stats=..., progress=...,
stop_ids=...)`` yields lists of new token ids, with mode "causal" (AR), "self-spec", or "diffusion"
(greedy block diffusion with the confidence-threshold commit gate of the reference's vLLM plugin,
qwen3_5_diffusion.py:449-632). With no `sampling`, decoding samples with SamplingParams() (temperature
1.0, top-k 50, top-p 0.95), the reference engine's default (engine.py:235); the diffusion mode is
greedy only.

Prompt cache (engine.py:1-10, 50-58, 140-200): each of up to `cache_slots` conversations keeps its
live cache (everything committed by its last generation) and, when the tokenizer has
``<|im_start|>``, snapshots right after the system block and right before the last ``<|im_start|>`` of
the previous prompt. A new prompt resumes from the longest of those that is a proper prefix of it
(the gated-delta state cannot rewind, so only these points are resumable); otherwise it takes an empty
or the least recently used slot. Caches grow to fit prompt + budget.

`model` is a checkpoint directory in the Hugging Face Qwen3.5 layout (trida_stack_amd.checkpoint; the
reference's model contract, inference/zoro-1/MODEL_CONTRACT.md:9-41), the name of a random-init shape,
or a prebuilt TridaRuntime. Nothing is downloaded.
"""
from __future__ import annotations

import contextlib
import itertools
import os
import threading
import time
from dataclasses import dataclass, field
from typing import Iterator, Optional, Union

from .decode import DecodeStats, SamplingParams, ar_generate, diffusion_generate, selfspec_generate
from .model import HybridConfig, TridaRuntime, build_runtime

MODES = ("causal", "self-spec", "diffusion")
SHAPES = {"random-4b": HybridConfig.four_b, "random-tiny": HybridConfig.tiny}


class IncrementalDetokenizer:
    """Streams the text of a growing list of token ids.

    Text is final up to `_flushed` ids. Each call decodes the unflushed ids together with up to
    `context` flushed ids before them (the ids a tokenizer needs to place spaces and merges), and
    returns what that decode adds to the decode of the context alone. An incomplete UTF-8 sequence
    at the end (the replacement character) holds the text back until a later id completes it."""

    def __init__(self, tokenizer, context: int = 4):
        self.tok = tokenizer
        self.context = int(context)
        self.ids: list = []
        self._flushed = 0

    def _text(self, ids: list) -> str:
        return self.tok.decode(ids, skip_special_tokens=False) if ids else ""

    def add(self, new_ids: list) -> str:
        self.ids.extend(int(t) for t in new_ids)
        lo = max(0, self._flushed - self.context)
        left = self._text(self.ids[lo: self._flushed])
        full = self._text(self.ids[lo:])
        if full.endswith("�") or not full.startswith(left):
            return ""
        self._flushed = len(self.ids)
        return full[len(left):]


def _is_prefix(head: list, seq: list) -> bool:
    return len(head) <= len(seq) and seq[: len(head)] == head


def _snap_tokens(snap) -> list:
    """Sequence 0's committed ids in a SeqCache.snapshot() tuple."""
    return snap[4][0]


@dataclass(eq=False)
class _Slot:
    """One conversation: its cache (one sequence), the snapshots it can rewind to (mark name ->
    SeqCache.snapshot()) and a least-recently-used stamp."""
    cache: object
    snaps: dict = field(default_factory=dict)
    used: int = 0

    def held(self) -> list:
        return self.cache.tokens[0]

    def resume_points(self):
        """(ids, snapshot) of every point this slot can continue from: the live cache (snapshot None),
        then each snapshot."""
        yield self.held(), None
        for snap in self.snaps.values():
            yield _snap_tokens(snap), snap

    def drop_stale(self) -> None:
        """Forgets the snapshots that are no longer a prefix of what the cache holds."""
        held = self.held()
        self.snaps = {name: snap for name, snap in self.snaps.items() if _is_prefix(_snap_tokens(snap), held)}


def _resume_marks(prompt: list, im_start: int) -> list:
    """(name, position) of the prompt's snapshot points, in prefill order: "system" at the second
    <|im_start|> when the prompt opens with one (the end of the system block), and "last" at the last
    <|im_start|> (before the generation header)."""
    starts = [i for i, t in enumerate(prompt) if t == im_start]
    marks = [("system", starts[1])] if len(starts) > 1 and starts[0] == 0 else []
    if starts:
        marks.append(("last", starts[-1]))
    return marks


def _load_tokenizer(path: Optional[str]):
    if not path:
        return None
    try:
        from transformers import AutoTokenizer

        return AutoTokenizer.from_pretrained(path, local_files_only=True)
    except Exception:  # noqa: BLE001 - a checkpoint without tokenizer files decodes token ids only
        return None


class Engine:
    def __init__(self, model: Union[str, TridaRuntime] = "random-4b", *, mode: str = "self-spec",
                 gen_block: Optional[int] = None, prefill_chunk: int = 512, prompt_cache: bool = True,
                 fused_gdn: Optional[bool] = None, cache_slots: int = 3, denoise_steps: int = 0, seed: int = 0,
                 device: str = "cuda:0", threshold: float = 0.9, canvas: int = 32, max_context: int = 8192,
                 tokenizer=None):
        """fused_gdn: True runs each GDN layer of a block as one launch (trida_gdn_fused_layer, bit-identical
        to the two-launch default, which measures faster on gfx950); None keeps the runtime's choice.
        max_context: the initial KV capacity of a slot (grown on demand)."""
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}")
        t = time.perf_counter()
        self.eos_ids: set = set()
        self.path = None
        if isinstance(model, TridaRuntime):
            self.rt = model
        elif os.path.isdir(str(model)):
            from .checkpoint import eos_ids_of, load_runtime

            self.path = str(model)
            self.rt = load_runtime(model, device=device)
            self.eos_ids = eos_ids_of(model)
        else:
            if model not in SHAPES:
                raise ValueError(f"unknown model {model!r}: not a checkpoint directory; shapes: {sorted(SHAPES)}")
            self.rt = build_runtime(SHAPES[model](), seed=seed, device=device)
        self.model_id = str(model) if not isinstance(model, TridaRuntime) else "runtime"
        self.rt.prefill_chunk = int(prefill_chunk)
        if fused_gdn is not None:
            self.rt.fused_gdn = bool(fused_gdn)
        self.tokenizer = tokenizer if tokenizer is not None else _load_tokenizer(self.path)
        self.im_start = None
        if self.tokenizer is not None:
            tid = self.tokenizer.convert_tokens_to_ids("<|im_start|>")
            if isinstance(tid, int) and tid >= 0 and tid != self.tokenizer.unk_token_id:
                self.im_start = tid
        self.mode = mode
        # self-spec block: N tokens per step (canvas 2N-1), or the draft block with denoise_steps > 0
        self.n = gen_block or (32 if denoise_steps else 4)
        self.denoise_steps = denoise_steps
        # block diffusion: canvas length and commit gate (the reference's defaults: 32 and 0.9)
        self.canvas, self.threshold = canvas, threshold
        self.mask_id = self.rt.mask_id
        self.use_prompt_cache = bool(prompt_cache)
        self.cache_slots = max(1, int(cache_slots))
        self.max_context = int(max_context)
        self._clock = itertools.count(1)
        self.reset_cache()
        self.lock = threading.Lock()
        self.last_stats: Optional[dict] = None
        self.load_s = time.perf_counter() - t

    # ------------------------------------------------------------------ caches
    @property
    def cache(self):
        return self.cur.cache

    def _new_cache(self):
        return self.rt.make_cache(1, max_len=self.max_context)

    def reset_cache(self) -> None:
        self.cur = _Slot(self._new_cache(), used=next(self._clock))
        self.slots = [self.cur]

    def cached_tokens(self) -> list:
        return [len(slot.held()) for slot in self.slots]

    def _best_resume(self, prompt: list):
        """(slot, snapshot or None) of the longest resumable point that is a proper, non-empty prefix of
        `prompt` (the first one found on equal lengths), or None."""
        best_len, best = 0, None
        for slot in self.slots:
            for ids, snap in slot.resume_points():
                if best_len < len(ids) < len(prompt) and _is_prefix(ids, prompt):
                    best_len, best = len(ids), (slot, snap)
        return best

    def _free_slot(self) -> _Slot:
        """An empty slot, else a new one while fewer than cache_slots exist, else the least recently
        used slot, emptied."""
        for slot in self.slots:
            if not slot.held():
                return slot
        if len(self.slots) < self.cache_slots:
            self.slots.append(_Slot(self._new_cache()))
            return self.slots[-1]
        slot = min(self.slots, key=lambda s: s.used)
        slot.cache, slot.snaps = self._new_cache(), {}
        return slot

    def _position_cache(self, prompt: list) -> None:
        """Makes self.cur the slot to continue `prompt` from: the one holding its longest reusable proper
        prefix (live, or a snapshot restored into the slot's cache), else a free slot (the prompt
        cache of engine.py:146-183)."""
        if not self.use_prompt_cache:
            self.reset_cache()
            return
        found = self._best_resume(prompt)
        if found is None:
            slot = self._free_slot()
        else:
            slot, snap = found
            if snap is not None:
                slot.cache.restore(snap)
            slot.drop_stale()
        slot.used = next(self._clock)
        self.cur = slot

    def _prefill_to_snapshot(self, prompt: list) -> None:
        """Prefills the prompt up to each snapshot point it has not reached yet and snapshots there
        (engine.py:185-198)."""
        if not self.use_prompt_cache or self.im_start is None:
            return
        for name, cut in _resume_marks(prompt, self.im_start):
            have = len(self.cur.held())
            if cut <= have:
                continue
            self.rt.prefill(self.cache, prompt[have:cut])
            self.cur.snaps[name] = self.cache.snapshot()

    # ------------------------------------------------------------------ generation
    def _rows_per_step(self, mode: str) -> int:
        if mode in ("causal", "ar"):
            return 1
        if mode == "diffusion":
            return self.canvas
        return self.n + 1 if self.denoise_steps else 2 * self.n - 1

    def _reserve(self, need: int) -> None:
        """Grows the current cache (in 1024-position steps) to hold `need` positions."""
        if need > self.cache.Lmax:
            self.rt.grow_cache(self.cache, -(-need // 1024) * 1024)

    @contextlib.contextmanager
    def _reporting(self, progress, total: int):
        """Routes the runtime's per-chunk prefill counts to progress(done, total) while active."""
        if progress is None:
            yield
            return
        done = 0

        def tick(k):
            nonlocal done
            done += k
            progress(done, total)

        self.rt.progress_cb = tick
        try:
            yield
        except BaseException:
            self.rt.progress_cb = None
            raise

    def _decoder(self, mode: str, prompt: list, max_tokens: int, eos_ids: set, sp: SamplingParams,
                 stats: DecodeStats):
        common = dict(max_new_tokens=max_tokens, eos_ids=eos_ids, sp=sp, stats=stats)
        if mode in ("causal", "ar"):
            return ar_generate(self.rt, self.cache, prompt, **common)
        if mode == "diffusion":
            return diffusion_generate(self.rt, self.cache, prompt, mask_id=self.mask_id, canvas=self.canvas,
                                      threshold=self.threshold, **common)
        return selfspec_generate(self.rt, self.cache, prompt, mask_id=self.mask_id, n=self.n,
                                 denoise_steps=self.denoise_steps, **common)

    def generate_ids(self, prompt: list, *, max_tokens: int = 2048, sampling: Optional[SamplingParams] = None,
                     mode: Optional[str] = None, stats: Optional[DecodeStats] = None, progress=None,
                     stop_ids: Optional[set] = None) -> Iterator[list]:
        """Yields lists of new token ids. Callers serialise calls (self.lock). progress(done, total) is
        called after each prefill chunk until the first tokens are out; stop_ids end the generation like
        EOS (engine.py:228-271)."""
        mode = mode or self.mode
        if sampling is None:
            sampling = SamplingParams(temperature=0.0) if mode == "diffusion" else SamplingParams()
        if mode == "diffusion" and not sampling.greedy:
            raise ValueError("diffusion mode decodes greedily (temperature 0)")
        stats = DecodeStats() if stats is None else stats
        started = time.perf_counter()
        self._position_cache(prompt)
        self._reserve(len(prompt) + max_tokens + 2 * self._rows_per_step(mode) + 16)
        reused = len(self.cur.held())
        with self._reporting(progress, len(prompt) - reused):
            self._prefill_to_snapshot(prompt)
        setup_s = time.perf_counter() - started
        gen = self._decoder(mode, prompt, max_tokens, self.eos_ids | set(stop_ids or ()), sampling, stats)
        try:
            first = True
            for chunk in gen:
                if first:  # the decoder's own prefill is done: no more progress reports
                    self.rt.progress_cb, first = None, False
                yield chunk
        finally:
            gen.close()
            self.rt.progress_cb = None
            stats.prefill_s += setup_s
            stats.reused_tokens = reused
            self.last_stats = stats.as_dict()

    # ------------------------------------------------------------------ text (checkpoints with a tokenizer)
    def _need_tokenizer(self):
        if self.tokenizer is None:
            raise ValueError("this model has no tokenizer; use generate_ids with token ids")
        return self.tokenizer

    def render(self, messages: list, tools: Optional[list] = None, enable_thinking: bool = True,
               **template_kwargs) -> str:
        """The chat template applied to `messages`, ending in the assistant generation header."""
        opts = dict(template_kwargs, add_generation_prompt=True, tokenize=False, enable_thinking=enable_thinking)
        if tools:
            opts["tools"] = tools
        return self._need_tokenizer().apply_chat_template(messages, **opts)

    def encode(self, text: str) -> list:
        return self._need_tokenizer().encode(text, add_special_tokens=False)

    def generate_text(self, prompt_text: str, **kw) -> Iterator[str]:
        """generate_ids over the encoded text, streamed back as text deltas."""
        stream = IncrementalDetokenizer(self._need_tokenizer())
        for ids in self.generate_ids(self.encode(prompt_text), **kw):
            piece = stream.add(ids)
            if piece:
                yield piece

    def warmup(self) -> None:
        """Runs one short greedy generation, so kernels, workspaces and graphs exist before the first
        request, then empties the caches."""
        if self.tokenizer is not None:
            prompt = self.encode("<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n")
        else:
            prompt = [1, 2, 3]
        with self.lock:
            for _ in self.generate_ids(prompt, max_tokens=8, sampling=SamplingParams(temperature=0.0)):
                pass
            self.reset_cache()
