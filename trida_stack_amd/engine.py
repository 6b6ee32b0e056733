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

import os
import threading
import time
from typing import Iterator, Optional, Union

from .decode import DecodeStats, SamplingParams, ar_generate, diffusion_generate, selfspec_generate
from .model import HybridConfig, TridaRuntime, build_runtime

MODES = ("causal", "self-spec", "diffusion")
SHAPES = {"random-4b": HybridConfig.four_b, "random-tiny": HybridConfig.tiny}


class IncrementalDetokenizer:
    """Text deltas of a growing id sequence, holding back an incomplete trailing character
    (engine.py:27-44)."""

    def __init__(self, tokenizer):
        self.tok = tokenizer
        self.ids: list = []
        self.prefix = 0
        self.read = 0

    def add(self, new_ids: list) -> str:
        self.ids.extend(new_ids)
        before = self.tok.decode(self.ids[self.prefix: self.read], skip_special_tokens=False)
        text = self.tok.decode(self.ids[self.prefix:], skip_special_tokens=False)
        if text.endswith("�"):
            return ""
        self.prefix, self.read = self.read, len(self.ids)
        return text[len(before):]


class _Slot:
    """One conversation's cache and its resumable snapshots (name -> SeqCache.snapshot())."""
    __slots__ = ("cache", "snaps", "used")

    def __init__(self, cache):
        self.cache, self.snaps, self.used = cache, {}, time.monotonic()


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
        self.cur = _Slot(self._new_cache())
        self.slots = [self.cur]

    def cached_tokens(self) -> list:
        return [len(s.cache.tokens[0]) for s in self.slots]

    def _position_cache(self, prompt: list) -> None:
        """Points self.cur at the slot holding the longest reusable proper prefix of `prompt` (its live
        tokens or a snapshot, restored), else at an empty slot, a new one, or the least recently used one
        (emptied) (engine.py:146-183)."""
        def usable(tokens):
            return 0 < len(tokens) < len(prompt) and prompt[: len(tokens)] == tokens

        if not self.use_prompt_cache:
            self.reset_cache()
            return
        best, best_slot, best_snap = 0, None, None
        for sl in self.slots:
            live = sl.cache.tokens[0]
            if usable(live) and len(live) > best:
                best, best_slot, best_snap = len(live), sl, None
            for snap in sl.snaps.values():
                if usable(snap[4][0]) and len(snap[4][0]) > best:
                    best, best_slot, best_snap = len(snap[4][0]), sl, snap
        if best_slot is not None:
            self.cur = best_slot
            if best_snap is not None:
                best_slot.cache.restore(best_snap)
            held = best_slot.cache.tokens[0]
            best_slot.snaps = {k: v for k, v in best_slot.snaps.items()
                               if len(v[4][0]) <= len(held) and held[: len(v[4][0])] == v[4][0]}
        elif any(len(sl.cache.tokens[0]) == 0 for sl in self.slots):
            self.cur = next(sl for sl in self.slots if len(sl.cache.tokens[0]) == 0)
        elif len(self.slots) < self.cache_slots:
            self.cur = _Slot(self._new_cache())
            self.slots.append(self.cur)
        else:
            self.cur = min(self.slots, key=lambda s: s.used)
            self.cur.cache, self.cur.snaps = self._new_cache(), {}
        self.cur.used = time.monotonic()

    def _prefill_to_snapshot(self, prompt: list) -> None:
        """Prefills up to the end of the system block and up to the last <|im_start|>, snapshotting at
        each (engine.py:185-198)."""
        if not self.use_prompt_cache or self.im_start is None:
            return
        starts = [i for i, t in enumerate(prompt) if t == self.im_start]
        marks = []
        if len(starts) >= 2 and starts[0] == 0:
            marks.append(("system", starts[1]))
        if starts:
            marks.append(("last", starts[-1]))
        for name, cut in marks:
            have = len(self.cache.tokens[0])
            if cut > have:
                self.rt.prefill(self.cache, prompt[have:cut])
                self.cur.snaps[name] = self.cache.snapshot()

    # ------------------------------------------------------------------ generation
    def generate_ids(self, prompt: list, *, max_tokens: int = 2048, sampling: Optional[SamplingParams] = None,
                     mode: Optional[str] = None, stats: Optional[DecodeStats] = None, progress=None,
                     stop_ids: Optional[set] = None) -> Iterator[list]:
        """Yields lists of new token ids. Callers serialise calls (self.lock). progress(done, total) is
        called after each prefill chunk; stop_ids end the generation like EOS (engine.py:200-271)."""
        eos_ids = self.eos_ids | set(stop_ids or ())
        mode = mode or self.mode
        if mode == "diffusion" and sampling is None:
            sampling = SamplingParams(temperature=0.0)
        sp = sampling or SamplingParams()
        stats = stats if stats is not None else DecodeStats()
        if mode == "diffusion" and not sp.greedy:
            raise ValueError("diffusion mode decodes greedily (temperature 0)")
        t = time.perf_counter()
        self._position_cache(prompt)
        step_rows = {"causal": 1, "ar": 1, "diffusion": self.canvas}.get(
            mode, (self.n + 1) if self.denoise_steps else (2 * self.n - 1))
        need = len(prompt) + max_tokens + 2 * step_rows + 16
        if need > self.cache.Lmax:
            self.rt.grow_cache(self.cache, -(-need // 1024) * 1024)
        reused = len(self.cache.tokens[0])
        if progress is not None:
            done = [0]
            total = len(prompt) - reused

            def _cb(k):
                done[0] += k
                progress(done[0], total)

            self.rt.progress_cb = _cb
        try:
            self._prefill_to_snapshot(prompt)
        except BaseException:
            self.rt.progress_cb = None
            raise
        pre_s = time.perf_counter() - t
        cache = self.cache
        if mode in ("causal", "ar"):
            gen = ar_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids, sp=sp, stats=stats)
        elif mode == "diffusion":
            gen = diffusion_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids,
                                     mask_id=self.mask_id, canvas=self.canvas, threshold=self.threshold, stats=stats,
                                     sp=sp)
        else:
            gen = selfspec_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids, sp=sp,
                                    mask_id=self.mask_id, n=self.n, stats=stats, denoise_steps=self.denoise_steps)
        try:
            for i, chunk in enumerate(gen):
                if i == 0:
                    self.rt.progress_cb = None
                yield chunk
        finally:
            gen.close()
            self.rt.progress_cb = None
            stats.prefill_s += pre_s
            stats.reused_tokens = reused
            self.last_stats = stats.as_dict()

    # ------------------------------------------------------------------ text (checkpoints with a tokenizer)
    def _need_tokenizer(self):
        if self.tokenizer is None:
            raise ValueError("this model has no tokenizer; use generate_ids with token ids")
        return self.tokenizer

    def render(self, messages: list, tools: Optional[list] = None, enable_thinking: bool = True,
               **template_kwargs) -> str:
        return self._need_tokenizer().apply_chat_template(messages, tools=tools or None, add_generation_prompt=True,
                                                          tokenize=False, enable_thinking=enable_thinking,
                                                          **template_kwargs)

    def encode(self, text: str) -> list:
        return self._need_tokenizer().encode(text, add_special_tokens=False)

    def generate_text(self, prompt_text: str, **kw) -> Iterator[str]:
        detok = IncrementalDetokenizer(self._need_tokenizer())
        for ids in self.generate_ids(self.encode(prompt_text), **kw):
            d = detok.add(ids)
            if d:
                yield d

    def warmup(self) -> None:
        """One short greedy generation (kernels, workspaces and graphs built), then empty caches."""
        with self.lock:
            p = self.encode("<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n") if self.tokenizer else [1, 2, 3]
            for _ in self.generate_ids(p, max_tokens=8, sampling=SamplingParams(temperature=0.0)):
                pass
            self.reset_cache()
