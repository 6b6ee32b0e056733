"""Decode configs: the YAML files the reference launcher maps each --mode to
(inference/zoro-1/serve.py:49-53; keys in inference/zoro-1/MODEL_CONTRACT.md:28-41 and
inference/zoro-1/configs/zoro1_self_spec_b15_g8.yaml:1-12), read into Engine keywords and
SamplingParams.

Supported values: variant bd_bidir_shift (the canvas algorithm, block_size = 2 * gen_block_size - 1),
causal_prefill true, use_spec_verify true, draft_mode strict_truncated (drafts drawn from the verifier's
truncated distribution, which is what the sampled self-spec here does). Any other value is rejected
rather than silently decoded another way. `threshold` is the diffusion mode's commit gate.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import yaml

from .decode import SamplingParams

CONFIGS = Path(__file__).resolve().parent / "configs"
# mode -> default decode config (the reference launcher's MODES table, serve.py:49-53)
MODE_CONFIGS = {"causal": None, "self-spec": "self_spec_b15_g8.yaml"}
KNOWN_KEYS = {"variant", "block_size", "gen_block_size", "mask_id", "causal_prefill", "temperature", "top_k",
              "top_p", "use_spec_verify", "draft_mode", "threshold"}


@dataclass
class DecodeConfig:
    variant: str = "bd_bidir_shift"
    block_size: Optional[int] = None
    gen_block_size: Optional[int] = None
    mask_id: Optional[int] = None
    causal_prefill: bool = True
    temperature: float = 1.0
    top_k: int = 50
    top_p: float = 0.95
    use_spec_verify: bool = True
    draft_mode: str = "strict_truncated"
    threshold: Optional[float] = None

    def sampling(self) -> SamplingParams:
        return SamplingParams(temperature=float(self.temperature), top_k=int(self.top_k), top_p=float(self.top_p))

    def engine_kwargs(self) -> dict:
        kw = {}
        if self.gen_block_size is not None:
            kw["gen_block"] = int(self.gen_block_size)
        if self.threshold is not None:
            kw["threshold"] = float(self.threshold)
        return kw

    def check_mask(self, mask_id: int) -> None:
        """The config's mask id must be the checkpoint's (MODEL_CONTRACT.md:24-27)."""
        if self.mask_id is not None and int(self.mask_id) != int(mask_id):
            raise ValueError(f"decode config mask_id {self.mask_id} != the model's mask id {mask_id}")


def parse(data: dict) -> DecodeConfig:
    unknown = set(data) - KNOWN_KEYS
    if unknown:
        raise ValueError(f"unknown decode config keys: {sorted(unknown)}")
    cfg = DecodeConfig(**{k: v for k, v in data.items()})
    if cfg.variant != "bd_bidir_shift":
        raise ValueError(f"decode variant {cfg.variant!r} is not supported (bd_bidir_shift is)")
    if cfg.gen_block_size is not None and cfg.block_size is not None \
            and int(cfg.block_size) != 2 * int(cfg.gen_block_size) - 1:
        raise ValueError("bd_bidir_shift needs block_size = 2 * gen_block_size - 1 "
                         f"(got {cfg.block_size} and {cfg.gen_block_size})")
    if not cfg.causal_prefill or not cfg.use_spec_verify:
        raise ValueError("only causal prefill with speculative verification is supported")
    if cfg.draft_mode != "strict_truncated":
        raise ValueError(f"draft_mode {cfg.draft_mode!r} is not supported (strict_truncated is)")
    return cfg


def load(path) -> DecodeConfig:
    with open(path) as f:
        data = yaml.safe_load(f) or {}
    if not isinstance(data, dict):
        raise ValueError(f"{path}: a decode config is a mapping")
    return parse(data)


def for_mode(mode: str) -> Optional[DecodeConfig]:
    name = MODE_CONFIGS.get(mode)
    return load(CONFIGS / name) if name else None
