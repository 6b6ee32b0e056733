"""Command line: ``python -m trida_stack_amd.cli --mode {causal,self-spec,diffusion}`` generates with the
engine and prints the tokens and decode stats as JSON. The --mode values are those of the reference
launcher (inference/zoro-1/serve.py:55-58, 199-201), and each mode reads its decode config as the
launcher does (serve.py:49-53): self-spec defaults to the model card's b15_g8 config (8 tokens per
step, temperature 1.0, top-k 20, top-p 0.95; trida_stack_amd/configs/self_spec_b15_g8.yaml); --config
names another YAML with the same keys, and --gen-block / --temperature / --top-k / --top-p override it.

--model is a checkpoint directory (Hugging Face Qwen3.5 layout) or a random-init shape name. With a
checkpoint that ships a tokenizer, --prompt takes text (the decoded continuation is printed too);
otherwise the prompt is --prompt-len random ids. --save-checkpoint DIR writes the random-init weights
of the shape as such a checkpoint directory and exits.
"""
from __future__ import annotations

import argparse
import json
import os
import random

from . import decode_config as DC
from .decode import SamplingParams
from .engine import MODES, SHAPES, Engine


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--mode", choices=MODES, default="self-spec")
    ap.add_argument("--model", default="random-tiny", help=f"checkpoint directory or one of {sorted(SHAPES)}")
    ap.add_argument("--config", default=None, help="decode config YAML (default: the mode's own)")
    ap.add_argument("--gen-block", type=int, default=None, help="tokens per self-spec step")
    ap.add_argument("--denoise-steps", type=int, default=0, help="> 0: draft-then-verify with this many passes")
    ap.add_argument("--temperature", type=float, default=None, help="0 decodes greedily")
    ap.add_argument("--top-k", type=int, default=None)
    ap.add_argument("--top-p", type=float, default=None)
    ap.add_argument("--banned", type=int, nargs="*", default=(), help="token ids never produced")
    ap.add_argument("--prefill-chunk", type=int, default=512)
    ap.add_argument("--no-prompt-cache", action="store_true")
    ap.add_argument("--cache-slots", type=int, default=3)
    ap.add_argument("--no-fused-gdn", action="store_true", help="two GDN launches per layer (the default here)")
    ap.add_argument("--prompt", default=None, help="prompt text (needs a checkpoint with a tokenizer)")
    ap.add_argument("--prompt-len", type=int, default=32)
    ap.add_argument("--max-tokens", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--save-checkpoint", default=None, help="write the random-init shape as a checkpoint here")
    args = ap.parse_args(argv)

    if args.save_checkpoint:
        from .checkpoint import save_checkpoint
        from .model import init_weights

        if args.model not in SHAPES:
            ap.error("--save-checkpoint needs a shape name as --model")
        cfg = SHAPES[args.model]()
        save_checkpoint(args.save_checkpoint, cfg, init_weights(cfg, seed=args.seed))
        print(json.dumps({"saved": os.path.abspath(args.save_checkpoint)}))
        return 0

    dcfg = DC.load(args.config) if args.config else DC.for_mode(args.mode)
    kw = dcfg.engine_kwargs() if dcfg else {}
    if args.gen_block is not None:
        kw["gen_block"] = args.gen_block
    sp = dcfg.sampling() if dcfg else SamplingParams()
    if args.temperature is not None:
        sp.temperature = args.temperature
    if args.top_k is not None:
        sp.top_k = args.top_k
    if args.top_p is not None:
        sp.top_p = args.top_p
    if args.mode == "diffusion" and args.temperature is None:
        sp.temperature = 0.0
    sp.seed = args.seed
    sp.banned = tuple(args.banned)
    eng = Engine(args.model, mode=args.mode, denoise_steps=args.denoise_steps, seed=args.seed,
                 prefill_chunk=args.prefill_chunk, prompt_cache=not args.no_prompt_cache,
                 cache_slots=args.cache_slots, fused_gdn=False if args.no_fused_gdn else None, **kw)
    if dcfg is not None and eng.path is not None:
        dcfg.check_mask(eng.mask_id)  # a checkpoint's mask token must match its decode config
    tok = eng.tokenizer
    if args.prompt is not None:
        if tok is None:
            ap.error("--prompt needs a checkpoint directory with a tokenizer")
        prompt = tok.encode(args.prompt)
    else:
        rng = random.Random(args.seed)
        prompt = [rng.randrange(0, eng.rt.cfg.vocab - 16) for _ in range(args.prompt_len)]
    toks = []
    with eng.lock:
        for chunk in eng.generate_ids(prompt, max_tokens=args.max_tokens, sampling=sp):
            toks.extend(chunk)
    out = {"mode": args.mode, "gen_block": eng.n, "temperature": sp.temperature, "top_k": sp.top_k,
           "top_p": sp.top_p, "tokens": toks, "stats": eng.last_stats}
    if tok is not None:
        out["text"] = tok.decode(toks)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
