"""Command line: ``python -m trida_stack_amd.cli --mode {causal,self-spec}`` generates with the
engine and prints the tokens and decode stats as JSON. The --mode values are those of the reference
launcher (inference/zoro-1/serve.py:55-58, 199-201).

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

from .engine import MODES, SHAPES, Engine


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--mode", choices=MODES, default="self-spec")
    ap.add_argument("--model", default="random-tiny", help=f"checkpoint directory or one of {sorted(SHAPES)}")
    ap.add_argument("--gen-block", type=int, default=None, help="tokens per self-spec step")
    ap.add_argument("--denoise-steps", type=int, default=0, help="> 0: draft-then-verify with this many passes")
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

    eng = Engine(args.model, mode=args.mode, gen_block=args.gen_block, denoise_steps=args.denoise_steps,
                 seed=args.seed)
    tok = None
    if args.prompt is not None:
        if eng.path is None:
            ap.error("--prompt needs a checkpoint directory with a tokenizer")
        from transformers import AutoTokenizer

        tok = AutoTokenizer.from_pretrained(eng.path, local_files_only=True)
        prompt = tok.encode(args.prompt)
    else:
        rng = random.Random(args.seed)
        prompt = [rng.randrange(0, eng.rt.cfg.vocab - 16) for _ in range(args.prompt_len)]
    toks = []
    with eng.lock:
        for chunk in eng.generate_ids(prompt, max_tokens=args.max_tokens):
            toks.extend(chunk)
    out = {"mode": args.mode, "tokens": toks, "stats": eng.last_stats}
    if tok is not None:
        out["text"] = tok.decode(toks)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
