"""Mode-switching generation engine (the drop-in surface of inference/zoro-1/mlx/trida_mlx/engine.py:60-80,
228-271): ``Engine(model, mode="self-spec", gen_block=N).generate_ids(prompt, mode=...)`` yields lists
of new token ids, with mode "causal" (AR), "self-spec", or "diffusion" (greedy block diffusion with the
confidence-threshold commit gate of the reference's vLLM plugin, qwen3_5_diffusion.py:449-632).

`model` is a checkpoint directory in the Hugging Face Qwen3.5 layout (trida_stack_amd.checkpoint; the
reference's model contract, inference/zoro-1/MODEL_CONTRACT.md:9-41), the name of a random-init shape,
or a prebuilt TridaRuntime. Nothing is downloaded. Prompts are token ids.
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


class Engine:
    def __init__(self, model: Union[str, TridaRuntime] = "random-4b", *, mode: str = "self-spec",
                 gen_block: Optional[int] = None, denoise_steps: int = 0, seed: int = 0, device: str = "cuda:0",
                 threshold: float = 0.9, canvas: int = 32):
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
        self.mode = mode
        # self-spec block: N tokens per step (canvas 2N-1), or the draft block with denoise_steps > 0
        self.n = gen_block or (32 if denoise_steps else 4)
        self.denoise_steps = denoise_steps
        # block diffusion: canvas length and commit gate (the reference's defaults: 32 and 0.9)
        self.canvas, self.threshold = canvas, threshold
        self.mask_id = self.rt.mask_id
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
        elif mode == "diffusion":
            if not sp.greedy:
                raise ValueError("diffusion mode decodes greedily (temperature 0)")
            cache = self.rt.make_cache(1, max_len=len(prompt) + max_tokens + self.canvas + 64)
            gen = diffusion_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids,
                                     mask_id=self.mask_id, canvas=self.canvas, threshold=self.threshold, stats=stats)
        else:
            gen = selfspec_generate(self.rt, cache, prompt, max_new_tokens=max_tokens, eos_ids=eos_ids, sp=sp,
                                    mask_id=self.mask_id, n=self.n, stats=stats, denoise_steps=self.denoise_steps)
        try:
            yield from gen
        finally:
            gen.close()
            self.last_stats = stats.as_dict()
