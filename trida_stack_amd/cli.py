"""Command line: ``python -m trida_stack_amd.cli --mode {causal,self-spec}`` generates from a random-id
prompt on a random-init model of a named shape and prints the tokens and decode stats as JSON. The
--mode values are those of the reference launcher (inference/zoro-1/serve.py:55-58, 199-201).
"""
from __future__ import annotations

import argparse
import json
import random

from .engine import MODES, SHAPES, Engine


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--mode", choices=MODES, default="self-spec")
    ap.add_argument("--model", choices=sorted(SHAPES), default="random-tiny")
    ap.add_argument("--gen-block", type=int, default=None, help="tokens per self-spec step")
    ap.add_argument("--denoise-steps", type=int, default=0, help="> 0: draft-then-verify with this many passes")
    ap.add_argument("--prompt-len", type=int, default=32)
    ap.add_argument("--max-tokens", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args(argv)
    eng = Engine(args.model, mode=args.mode, gen_block=args.gen_block, denoise_steps=args.denoise_steps,
                 seed=args.seed)
    rng = random.Random(args.seed)
    prompt = [rng.randrange(0, eng.rt.cfg.vocab - 16) for _ in range(args.prompt_len)]
    toks = []
    with eng.lock:
        for chunk in eng.generate_ids(prompt, max_tokens=args.max_tokens):
            toks.extend(chunk)
    print(json.dumps({"mode": args.mode, "tokens": toks, "stats": eng.last_stats}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
