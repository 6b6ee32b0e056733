"""Mode-switching generation engine (the drop-in surface of inference/zoro-1/mlx/trida_mlx/engine.py:60-80,
228-271): ``Engine(model, mode="self-spec", gen_block=N).generate_ids(prompt, mode=...)`` yields lists
of new token ids, with mode "causal" (AR) or "self-spec".

Models are random-init hybrids of a named shape (no checkpoint download); a prebuilt TridaRuntime can
be passed instead. Prompts are token ids.
"""
from __future__ import annotations

import threading
import time
from typing import Iterator, Optional, Union

from .decode import DecodeStats, SamplingParams, ar_generate, selfspec_generate
from .model import HybridConfig, TridaRuntime, build_runtime

MODES = ("causal", "self-spec")
SHAPES = {"random-4b": HybridConfig.four_b, "random-tiny": HybridConfig.tiny}


class Engine:
    def __init__(self, model: Union[str, TridaRuntime] = "random-4b", *, mode: str = "self-spec",
                 gen_block: Optional[int] = None, denoise_steps: int = 0, seed: int = 0, device: str = "cuda:0"):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}")
        t = time.perf_counter()
        if isinstance(model, TridaRuntime):
            self.rt = model
        else:
            if model not in SHAPES:
                raise ValueError(f"unknown model {model!r}; known: {sorted(SHAPES)}")
            self.rt = build_runtime(SHAPES[model](), seed=seed, device=device)
        self.mode = mode
        # self-spec block: N tokens per step (canvas 2N-1), or the draft block with denoise_steps > 0
        self.n = gen_block or (32 if denoise_steps else 4)
        self.denoise_steps = denoise_steps
        self.mask_id = self.rt.mask_id
        self.eos_ids: set = set()
        self.lock = threading.Lock()
        self.last_stats: Optional[dict] = None
        self.load_s = time.perf_counter() - t

    def generate_ids(self, prompt: list, *, max_tokens: int = 2048, sampling: Optional[SamplingParams] = None,
                     mode: Optional[str] = None, stats: Optional[DecodeStats] = None,
                     stop_ids: Optional[set] = None) -> Iterator[list]:
        eos_ids = self.eos_ids | set(stop_ids or ())
        sp = sampling or SamplingParams(temperature=0.0)
        mode = mode or self.mode
        stats = stats if stats is not None else DecodeStats()
        margin = 2 * self.n + 8 if not self.denoise_steps else (self.n + 1) * 2
        cache = self.rt.make_cache(1, max_len=len(prompt) + max_tokens * (1 if mode == "causal" else 2) + margin + 64)
        if mode in ("causal", "ar"):
            gen = ar_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids, sp=sp, stats=stats)
        else:
            gen = selfspec_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids, sp=sp,
                                    mask_id=self.mask_id, n=self.n, stats=stats, denoise_steps=self.denoise_steps)
        try:
            yield from gen
        finally:
            gen.close()
            self.last_stats = stats.as_dict()
