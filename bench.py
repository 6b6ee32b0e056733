"""Benchmark of the MI355X self-speculative decode step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload accept]

Prints ONE JSON line (rank 0). One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "accepted tok/s (bs1, bs64) on 4B-shape hybrid; verify-step µs; % HBM peak"
HBM_PEAK_GBS = 8000.0


def _events_time_ms(fn, iters: int) -> float:
    """Average ms per call of fn, from HIP events on the current stream, with the calls captured in
    one HIP graph so the launch gaps of a host loop do not count."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm: workspaces and allocator pools exist before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


# ------------------------------------------------------------------------------ greedy acceptance
def bench_accept(args):
    import numpy as np
    import torch

    from trida_stack_amd import kernels, workloads

    dev = torch.device("cuda:0")
    B, K, V, ctx = 1, 32, 151936, 4096
    w = workloads.greedy_accept_inputs(seed=0, batch=B, block=K, vocab=V, ctx=ctx)
    lg, dr, cl = w["logits"].to(dev), w["drafts"].to(dev), w["ctx_len"].to(dev)
    fn = lambda: kernels.greedy_accept(lg, dr, ctx_len=cl, splits=args.splits)
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = fn()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kern_ms = _events_time_ms(fn, 200)
    nbytes = B * (K + 1) * V * 4
    achieved = nbytes / (kern_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        from oracle import accept as A

        lg_np, dr_np, cl_np = w["logits"].numpy(), w["drafts"].numpy(), w["ctx_len"].numpy()
        A.greedy_accept(lg_np, dr_np, ctx_len=cl_np)
        reps, t = 0, time.perf_counter()
        while time.perf_counter() - t < 3.0:
            A.greedy_accept(lg_np, dr_np, ctx_len=cl_np)
            reps += 1
        cpu_us = (time.perf_counter() - t) / reps * 1e6
        cpu = {"value": round(cpu_us, 2), "unit": "us per verify step", "cores": 1, "kind": "port",
               "sample": f"{reps} oracle greedy_accept calls on the same [1,33,151936] fp32 logits (numpy)"}
    n_acc = int(out[1][0])
    return {
        "metric": METRIC, "value": round(kern_ms * 1e3, 3), "unit": "us per greedy verify step (kernel)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "greedy acceptance, batch 1, block 32, vocab 151936, ctx 4096",
                   "n_acc": n_acc},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="accept", choices=["accept"])
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the step shards by "
              "sequence; see the sharding notes)", file=sys.stderr)
        sys.exit(2)
    res = {"accept": bench_accept}[args.workload](args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
