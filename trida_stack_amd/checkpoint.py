"""Hugging Face checkpoints of the Qwen3.5-architecture hybrid (Zoro-1 / Trida layout).

Follows the reference's loader (inference/zoro-1/mlx/trida_mlx/model.py:44-139) and its model contract
(inference/zoro-1/MODEL_CONTRACT.md:9-41): a directory with ``config.json`` (the text model's fields,
possibly nested under ``text_config``), bf16 ``*.safetensors`` weights under the transformers
Qwen3.5 names, and the mask token id in ``block_diffusion.json``.

Conventions carried over unchanged (the runtime already computes with them): RMSNorm weights are
zero-centred (y = x_hat * (1 + w)) except the GDN output norm, depthwise conv weights are [C, 1, K] on
disk, ``A_log`` stays fp32, the attention q projection interleaves [q | gate] per head, and a tied LM
head is the embedding (a shipped ``lm_head.weight`` is then ignored, as HF and vLLM do;
inference/zoro-1/mlx/trida_mlx/model.py:97-107).

The runtime packs projections that read the same input: attention ``[q|gate, k, v]``, GDN
``[qkv, z, b, a]`` and FFN ``[gate, up]``, each one GEMM.
"""
from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Dict, Optional, Tuple

import torch

from .model import DEFAULT_MASK_ID, HybridConfig, TridaRuntime

# files in a checkpoint directory that hold other heads, not the language model
_OTHER_HEADS = ("decision_head.safetensors", "jev_head.safetensors")


def _text_config(cfg: dict) -> dict:
    """The language model's fields (multimodal checkpoints nest them under text_config)."""
    text = dict(cfg.get("text_config", cfg))
    if "tie_word_embeddings" not in text and "tie_word_embeddings" in cfg:
        text["tie_word_embeddings"] = cfg["tie_word_embeddings"]
    return text


def config_from_hf(cfg: dict, mask_id: int = DEFAULT_MASK_ID) -> HybridConfig:
    """HybridConfig from a checkpoint's config.json (transformers Qwen3_5TextConfig field names)."""
    t = _text_config(cfg)
    rope = t.get("rope_parameters") or {}
    n_layers = int(t["num_hidden_layers"])
    layer_types = t.get("layer_types")
    if layer_types is None:
        interval = int(t.get("full_attention_interval", 4))
        layer_types = ["full_attention" if (i + 1) % interval == 0 else "linear_attention" for i in range(n_layers)]
    if len(layer_types) != n_layers or any(x not in ("full_attention", "linear_attention") for x in layer_types):
        raise ValueError(f"layer_types must list {n_layers} 'full_attention' / 'linear_attention' entries")
    return HybridConfig(
        hidden=int(t["hidden_size"]), n_layers=n_layers, intermediate=int(t["intermediate_size"]),
        vocab=int(t["vocab_size"]), lin_k_heads=int(t["linear_num_key_heads"]),
        lin_v_heads=int(t["linear_num_value_heads"]), lin_k_dim=int(t["linear_key_head_dim"]),
        lin_v_dim=int(t["linear_value_head_dim"]), conv_kernel=int(t.get("linear_conv_kernel_dim", 4)),
        n_heads=int(t["num_attention_heads"]), n_kv_heads=int(t["num_key_value_heads"]),
        head_dim=int(t.get("head_dim", 256)),
        rotary_frac=float(rope.get("partial_rotary_factor", t.get("partial_rotary_factor", 0.25))),
        rope_theta=float(rope.get("rope_theta", t.get("rope_theta", 1.0e7))),
        rms_eps=float(t.get("rms_norm_eps", 1e-6)), mask_id=int(mask_id),
        tie_embeddings=bool(t.get("tie_word_embeddings", False)), layer_types=tuple(layer_types))


def config_to_hf(cfg: HybridConfig) -> dict:
    """config.json fields of a text-only Qwen3.5 checkpoint for cfg."""
    return {
        "architectures": ["Qwen3_5ForCausalLM"], "model_type": "qwen3_5_text",
        "hidden_size": cfg.hidden, "num_hidden_layers": cfg.n_layers, "intermediate_size": cfg.intermediate,
        "vocab_size": cfg.vocab, "linear_num_key_heads": cfg.lin_k_heads, "linear_num_value_heads": cfg.lin_v_heads,
        "linear_key_head_dim": cfg.lin_k_dim, "linear_value_head_dim": cfg.lin_v_dim,
        "linear_conv_kernel_dim": cfg.conv_kernel, "num_attention_heads": cfg.n_heads,
        "num_key_value_heads": cfg.n_kv_heads, "head_dim": cfg.head_dim, "hidden_act": "silu",
        "rms_norm_eps": cfg.rms_eps, "tie_word_embeddings": cfg.tie_embeddings,
        "layer_types": ["full_attention" if cfg.is_attention(i) else "linear_attention" for i in range(cfg.n_layers)],
        "rope_parameters": {"rope_type": "default", "rope_theta": cfg.rope_theta,
                            "partial_rotary_factor": cfg.rotary_frac},
        "max_position_embeddings": 262144, "torch_dtype": "bfloat16",
    }


def mask_id_of(path: Path, cfg: dict, tokenizer=None) -> int:
    """The mask token id: block_diffusion.json, then config.json, then the tokenizer's <|mask|>, then
    the Zoro-1 default (inference/zoro-1/mlx/trida_mlx/model.py:126-138)."""
    bd = Path(path) / "block_diffusion.json"
    if bd.is_file():
        return int(json.loads(bd.read_text())["mask_id"])
    if "mask_id" in cfg:
        return int(cfg["mask_id"])
    if tokenizer is not None:
        tid = tokenizer.convert_tokens_to_ids("<|mask|>")
        if isinstance(tid, int) and tid >= 0 and tid != getattr(tokenizer, "unk_token_id", None):
            return tid
    return DEFAULT_MASK_ID


def _canonical(name: str) -> str:
    """HF text-model key from a text-only or multimodal checkpoint key."""
    for pre, rep in (("model.language_model.", "model."), ("language_model.model.", "model."),
                     ("language_model.", "")):
        if name.startswith(pre):
            return rep + name[len(pre):]
    return name


def _is_language_key(name: str) -> bool:
    return name.startswith("model.") or name == "lm_head.weight"


def hf_to_runtime(hf: Dict[str, torch.Tensor], cfg: HybridConfig, dtype=torch.bfloat16) -> Dict[str, torch.Tensor]:
    """Runtime weights (packed projections) from HF-named tensors. Missing or misshapen tensors raise."""
    def get(k, shape=None):
        if k not in hf:
            raise KeyError(f"checkpoint has no tensor {k!r}")
        t = hf[k]
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{k}: shape {tuple(t.shape)}, expected {tuple(shape)}")
        return t

    h, I, V = cfg.hidden, cfg.intermediate, cfg.vocab
    bf = lambda t: t.to(dtype).contiguous()
    w = {"embed": bf(get("model.embed_tokens.weight", (V, h))), "final_norm": bf(get("model.norm.weight", (h,)))}
    if not cfg.tie_embeddings:
        w["lm_head"] = bf(get("lm_head.weight", (V, h)))
    for i in range(cfg.n_layers):
        P, p = f"model.layers.{i}.", f"l{i}."
        w[p + "in_norm"] = bf(get(P + "input_layernorm.weight", (h,)))
        w[p + "post_norm"] = bf(get(P + "post_attention_layernorm.weight", (h,)))
        w[p + "w_gu"] = bf(torch.cat([get(P + "mlp.gate_proj.weight", (I, h)), get(P + "mlp.up_proj.weight", (I, h))]))
        w[p + "w_down"] = bf(get(P + "mlp.down_proj.weight", (h, I)))
        if cfg.is_attention(i):
            A = P + "self_attn."
            Dq, Dkv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
            w[p + "w_qkv"] = bf(torch.cat([get(A + "q_proj.weight", (2 * Dq, h)), get(A + "k_proj.weight", (Dkv, h)),
                                           get(A + "v_proj.weight", (Dkv, h))]))
            w[p + "q_norm"] = bf(get(A + "q_norm.weight", (cfg.head_dim,)))
            w[p + "k_norm"] = bf(get(A + "k_norm.weight", (cfg.head_dim,)))
            w[p + "w_o"] = bf(get(A + "o_proj.weight", (h, Dq)))
        else:
            G, Hv = P + "linear_attn.", cfg.lin_v_heads
            w[p + "w_in"] = bf(torch.cat([get(G + "in_proj_qkv.weight", (cfg.conv_dim, h)),
                                          get(G + "in_proj_z.weight", (cfg.value_dim, h)),
                                          get(G + "in_proj_b.weight", (Hv, h)), get(G + "in_proj_a.weight", (Hv, h))]))
            w[p + "conv_w"] = bf(get(G + "conv1d.weight", (cfg.conv_dim, 1, cfg.conv_kernel)).reshape(cfg.conv_dim, -1))
            w[p + "A_log"] = get(G + "A_log", (Hv,)).float().contiguous()
            w[p + "dt_bias"] = get(G + "dt_bias", (Hv,)).float().contiguous()
            w[p + "gnorm"] = bf(get(G + "norm.weight", (cfg.lin_v_dim,)))
            w[p + "w_out"] = bf(get(G + "out_proj.weight", (h, cfg.value_dim)))
    return w


def runtime_to_hf(w: Dict[str, torch.Tensor], cfg: HybridConfig) -> Dict[str, torch.Tensor]:
    """HF-named tensors from runtime weights (the inverse of hf_to_runtime; bf16 except A_log)."""
    h, I = cfg.hidden, cfg.intermediate
    bf = lambda t: t.to(torch.bfloat16).contiguous().cpu()
    hf = {"model.embed_tokens.weight": bf(w["embed"]), "model.norm.weight": bf(w["final_norm"])}
    # shipped alongside a tied head too, as Zoro-1 does (a separate copy: safetensors stores no aliases)
    hf["lm_head.weight"] = bf(w["lm_head"]) if "lm_head" in w else hf["model.embed_tokens.weight"].clone()
    for i in range(cfg.n_layers):
        P, p = f"model.layers.{i}.", f"l{i}."
        hf[P + "input_layernorm.weight"] = bf(w[p + "in_norm"])
        hf[P + "post_attention_layernorm.weight"] = bf(w[p + "post_norm"])
        gu = w[p + "w_gu"]
        hf[P + "mlp.gate_proj.weight"], hf[P + "mlp.up_proj.weight"] = bf(gu[:I]), bf(gu[I:])
        hf[P + "mlp.down_proj.weight"] = bf(w[p + "w_down"])
        if cfg.is_attention(i):
            A = P + "self_attn."
            Dq, Dkv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
            q, k, v = torch.split(w[p + "w_qkv"], [2 * Dq, Dkv, Dkv])
            hf[A + "q_proj.weight"], hf[A + "k_proj.weight"], hf[A + "v_proj.weight"] = bf(q), bf(k), bf(v)
            hf[A + "q_norm.weight"], hf[A + "k_norm.weight"] = bf(w[p + "q_norm"]), bf(w[p + "k_norm"])
            hf[A + "o_proj.weight"] = bf(w[p + "w_o"])
        else:
            G, Hv = P + "linear_attn.", cfg.lin_v_heads
            qkv, z, b, a = torch.split(w[p + "w_in"], [cfg.conv_dim, cfg.value_dim, Hv, Hv])
            hf[G + "in_proj_qkv.weight"], hf[G + "in_proj_z.weight"] = bf(qkv), bf(z)
            hf[G + "in_proj_b.weight"], hf[G + "in_proj_a.weight"] = bf(b), bf(a)
            hf[G + "conv1d.weight"] = bf(w[p + "conv_w"]).reshape(cfg.conv_dim, 1, cfg.conv_kernel)
            hf[G + "A_log"] = w[p + "A_log"].float().contiguous().cpu()
            hf[G + "dt_bias"] = bf(w[p + "dt_bias"])
            hf[G + "norm.weight"] = bf(w[p + "gnorm"])
            hf[G + "out_proj.weight"] = bf(w[p + "w_out"])
    return hf


def load_weights(path, device="cpu") -> Tuple[HybridConfig, Dict[str, torch.Tensor], dict]:
    """(config, runtime weights on `device`, config.json) of a checkpoint directory. Reads every
    *.safetensors file except the decision / jev heads, keeps the language model's tensors only."""
    from safetensors import safe_open

    path = Path(path)
    cfg_json = json.loads((path / "config.json").read_text())
    cfg = config_from_hf(cfg_json, mask_id_of(path, cfg_json))
    hf: Dict[str, torch.Tensor] = {}
    files = sorted(f for f in path.glob("*.safetensors") if f.name not in _OTHER_HEADS)
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {path}")
    dev = str(device)
    for f in files:
        with safe_open(str(f), framework="pt", device=dev) as fh:
            for k in fh.keys():
                name = _canonical(k)
                if _is_language_key(name):
                    hf[name] = fh.get_tensor(k)
    if cfg.tie_embeddings and "lm_head.weight" in hf and "model.embed_tokens.weight" in hf:
        head, emb = hf.pop("lm_head.weight"), hf["model.embed_tokens.weight"]
        if head.shape == emb.shape and not torch.equal(head, emb):
            print("[trida] warning: config ties embeddings but lm_head.weight differs from embed_tokens; "
                  "using embed_tokens (as HF / vLLM do)", flush=True)
    return cfg, hf_to_runtime(hf, cfg), cfg_json


def load_runtime(path, device="cuda:0") -> TridaRuntime:
    """A TridaRuntime over a checkpoint directory (weights read straight to `device`)."""
    cfg, w, _ = load_weights(path, device=device)
    return TridaRuntime(cfg, w, device=device)


def eos_ids_of(path) -> set:
    """End-of-sequence ids from generation_config.json (int or list), empty when absent."""
    f = Path(path) / "generation_config.json"
    if not f.is_file():
        return set()
    e = json.loads(f.read_text()).get("eos_token_id")
    if e is None:
        return set()
    return {int(x) for x in (e if isinstance(e, list) else [e])}


def save_checkpoint(path, cfg: HybridConfig, w: Dict[str, torch.Tensor], eos_ids=None) -> Path:
    """Writes cfg and runtime weights as a text-only HF checkpoint directory (config.json,
    model.safetensors, block_diffusion.json, generation_config.json) that load_weights and
    transformers' Qwen3_5ForCausalLM both read."""
    from safetensors.torch import save_file

    path = Path(path)
    os.makedirs(path, exist_ok=True)
    save_file(runtime_to_hf(w, cfg), str(path / "model.safetensors"), metadata={"format": "pt"})
    (path / "config.json").write_text(json.dumps(config_to_hf(cfg), indent=2))
    (path / "block_diffusion.json").write_text(json.dumps({"mask_id": cfg.mask_id}))
    if eos_ids:
        (path / "generation_config.json").write_text(json.dumps({"eos_token_id": sorted(eos_ids)}))
    return path
