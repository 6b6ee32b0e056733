"""Benchmark of the MI355X self-speculative decode step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload e2e|e2e64|gdr|accept|sample|attn|gemm]

Prints ONE JSON line (rank 0). One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "accepted tok/s (bs1, bs64) on 4B-shape hybrid; verify-step µs; % HBM peak"
HBM_PEAK_GBS = 8000.0


def _measured_traffic(*keys):
    """HBM bytes per call: the sum over `keys` of the calibrated rocprofv3 FETCH_SIZE / WRITE_SIZE bytes
    per dispatch in profiles/hbm_traffic.md (measured on MI355X by two counter passes over this
    bench), or None when that table or a key is missing."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.md")
    try:
        with open(path) as f:
            lines = f.read().splitlines()
    except OSError:
        return None
    vals = {}
    for ln in lines:
        parts = [p.strip() for p in ln.split("|")]
        if len(parts) > 6 and parts[5].isdigit():
            vals[parts[1]] = int(parts[5])
    try:
        return sum(vals[k] for k in keys)
    except KeyError:
        return None


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
    at_scale = _greedy_accept_at_scale(dev, K)
    return {
        "metric": METRIC, "value": round(kern_ms * 1e3, 3), "unit": "us per greedy verify step (kernel)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "greedy acceptance, batch 1, block 32, vocab 151936, ctx 4096",
                   "n_acc": n_acc},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _measured_traffic("accept_split_argmax", "accept_finalize")},
        "at_scale": at_scale,
        "cpu_baseline": cpu,
    }


def _greedy_accept_at_scale(dev, K):
    """The same two kernels at batch 64 over the 4B-shape vocabulary (248320): the verify logits in the
    runtime's bf16 layout (1.05 GB) and in fp32 (2.1 GB). At 20 MB (batch 1) a launch is latency-bound;
    here the HBM stream dominates."""
    import torch

    from trida_stack_amd import kernels

    B, V = 64, 248320
    g = torch.Generator(device=dev).manual_seed(1)
    drafts = torch.randint(0, V, (B, K), generator=g, device=dev)
    ctx = torch.full((B,), 4096, dtype=torch.int64, device=dev)
    res = {}
    for dt, esz in ((torch.bfloat16, 2), (torch.float32, 4)):
        lg = (torch.randn(B, K + 1, V, generator=g, device=dev) * 2).to(dt)
        fn = lambda: kernels.greedy_accept(lg, drafts, ctx_len=ctx)
        for _ in range(3):
            fn()
        us = _events_time_ms(fn, 20) * 1e3
        nbytes = B * (K + 1) * V * esz
        gbs = nbytes / (us * 1e-6) / 1e9
        res[str(dt).replace("torch.", "")] = {"us": round(us, 1), "bytes": nbytes, "GBps": round(gbs, 1),
                                              "frac": round(gbs / HBM_PEAK_GBS, 4)}
        del lg
    return {"workload": f"greedy acceptance, batch {B}, {K + 1} verify rows, vocab {V}", **res}


# ------------------------------------------------------------------------------ sampled acceptance
def bench_sample(args):
    """Rejection-sampling acceptance of one bs64 verify step: p logits [64, 33, 248320] fp32 ~ N(0, 4),
    draft distributions q [64, 32, 248320] fp32 (truncated probabilities of perturbed logits), drafts
    drawn from q, temperature 0.7, top-p 0.95, seeded uniforms."""
    import torch

    from trida_stack_amd import kernels

    dev = torch.device("cuda:0")
    B, K, V, T, TOP_P = 64, 32, 248320, 0.7, 0.95
    g = torch.Generator(device=dev).manual_seed(0)
    pl = torch.randn(B, K + 1, V, generator=g, device=dev) * 2
    ql = pl[:, :K] + torch.randn(B, K, V, generator=g, device=dev) * 0.3
    q = kernels.truncated_probs(ql, kernels.truncate_stats(ql, temperature=T, top_p=TOP_P), temperature=T)
    del ql
    drafts = torch.multinomial(q.reshape(-1, V), 1, generator=g).reshape(B, K)
    ua = torch.rand(B, K, generator=g, device=dev)
    us = torch.rand(B, generator=g, device=dev)
    ctx = torch.full((B,), 4096, dtype=torch.int64, device=dev)
    out = [torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int64, device=dev),
           torch.empty(B, dtype=torch.int64, device=dev), None, torch.empty(B, dtype=torch.int32, device=dev)]
    fn = lambda: kernels.sample_accept(pl, q, drafts, ua, us, temperature=T, top_p=TOP_P, ctx_len=ctx, out=out)
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        fn()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kern_ms = _events_time_ms(fn, 20)
    passes = kernels.truncate_stats(pl, temperature=T, top_p=TOP_P, want_passes=True)[4]
    one_pass = float((passes == 4).float().mean())  # 4 streamed quarter-rows = one pass
    mean_passes = float(passes.float().mean()) / 4
    n_acc = out[0].cpu()
    # Bytes this algorithm must read: the verify rows it evaluates (the first group of G0 rows of every
    # sequence, all K + 1 rows of the sequences that accept past it), then the correction row of p and
    # q per sequence. The reference evaluates every verify row (B * (K + 1) * V * 4 bytes + the
    # correction rows); that figure is reported alongside.
    G0 = min(K + 1, max(8, -(-512 // B)))
    rows_read = int(sum(G0 if int(n) < G0 else K + 1 for n in n_acc))
    nbytes = rows_read * V * 4 + B * 2 * V * 4
    ref_bytes = B * (K + 1) * V * 4 + B * 2 * V * 4
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        from oracle import accept as A

        ns = 2
        p_np, q_np = pl[:ns].cpu().numpy(), q[:ns].cpu().numpy()
        d_np, ua_np, us_np = drafts[:ns].cpu().numpy(), ua[:ns].cpu().numpy(), us[:ns].cpu().numpy()
        t = time.perf_counter()
        A.rejection_accept(p_np, q_np, d_np, ua_np, us_np, temperature=T, top_p=TOP_P)
        per_seq = (time.perf_counter() - t) / ns
        cpu = {"value": round(per_seq * B * 1e3, 1), "unit": "ms per bs64 verify step (extrapolated)", "cores": 1,
               "kind": "port", "sample": f"oracle rejection_accept on {ns} of the 64 sequences (33 x 248320 fp32 "
                                         f"rows each, numpy float64), x {B // ns}"}
    return {
        "metric": METRIC, "value": round(kern_ms * 1e3, 1), "unit": "us per bs64 sampled verify step (kernels)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "sampled acceptance, batch 64, block 32 (33 verify rows), vocab 248320, temperature "
                               "0.7, top-p 0.95, q as full-vocabulary fp32 probabilities",
                   "one_pass_rows": round(one_pass, 3), "mean_passes_per_row": round(mean_passes, 3),
                   "mean_n_acc": round(float(n_acc.float().mean()), 2), "verify_rows_read": rows_read,
                   "bytes_read": nbytes, "reference_bytes": ref_bytes,
                   "reference_equivalent_GBps": round(ref_bytes / (kern_ms * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _measured_traffic("sample_truncate_g0", "sample_truncate_g1", "sample_resid_sums")},
        "cpu_baseline": cpu,
    }


# ------------------------------------------------------------------------------ canvas attention
def bench_attn(args):
    """Canvas attention of one verify block: q [1, 32, 16, 256] bf16 against a bf16 KV cache of 8192
    prefix + 32 block keys per kv head (4 kv heads), verify (causal block) and draft (bidirectional
    block) masks, then the crop to 8192 + a."""
    import torch

    from trida_stack_amd import kernels

    dev = torch.device("cuda:0")
    B, T, Hq, Hkv, D, P = 1, 32, 16, 4, 256, 8192
    L = P + T
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, T, Hq, D, generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn(B, Hkv, L, D, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(B, Hkv, L, D, generator=g, device=dev).to(torch.bfloat16)
    plen = torch.full((B,), P, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    res = {}
    for name, mode in (("verify", kernels.MASK_VERIFY), ("draft", kernels.MASK_DRAFT)):
        fn = lambda: kernels.attn_canvas(q, kc, vc, plen, mask_mode=mode, out=out, max_keys=L, splits=args.splits)
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
        res[name] = (_events_time_ms(fn, 200), wall_ms)
    # crop to 8192 + a: a device-side length update (the cache keeps its memory)
    a = 17
    crop = lambda: plen.fill_(P + a)
    crop_ms = _events_time_ms(crop, 200)
    plen.fill_(P)
    nbytes = 2 * L * Hkv * D * 2 + 2 * B * T * Hq * D * 2
    flops = 4 * Hq * T * L * D
    kern_ms = res["verify"][0]
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        from oracle import attention as OA

        qc, kk, vv = q.float().cpu(), kc.float().cpu(), vc.float().cpu()
        pl = [P]
        OA.canvas_attention(qc, kk, vv, pl, kernels.MASK_VERIFY)
        t = time.perf_counter()
        reps = 0
        while time.perf_counter() - t < 3.0:
            OA.canvas_attention(qc, kk, vv, pl, kernels.MASK_VERIFY)
            reps += 1
        cpu = {"value": round((time.perf_counter() - t) / reps * 1e6, 1), "unit": "us per verify attention",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{reps} oracle canvas_attention calls (torch fp32 on the host) on the same inputs"}
    return {
        "metric": METRIC, "value": round(kern_ms * 1e3, 2), "unit": "us per verify-block attention (kernels)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res["verify"][1], 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "canvas attention, 32 block rows, 16 q / 4 kv heads, d 256, ctx 8192 + 32",
                   "draft_us": round(res["draft"][0] * 1e3, 2), "crop_us": round(crop_ms * 1e3, 2),
                   "tflops": round(flops / (kern_ms * 1e-3) / 1e12, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _measured_traffic("attn_partial", "attn_combine")},
        "cpu_baseline": cpu,
    }


# ------------------------------------------------------------------------------ end-to-end (config 4)
PROMPT_LEN, BLOCK, DENOISE = 2048, 32, 4


def _cpu_cache(cfg, ctx: int, prompt_tail, seed: int = 1):
    """An oracle cache holding a synthetic ctx-token context: random KV entries and GDN states of the
    real shapes instead of a CPU prefill (which would take minutes at 4B scale)."""
    import torch

    from oracle import model as OM

    cache = OM.CpuCache()
    g = torch.Generator().manual_seed(seed)
    for i in range(cfg.n_layers):
        if cfg.is_attention(i):
            shape = (cfg.n_kv_heads, ctx, cfg.head_dim)
            cache.kv[i] = (torch.randn(*shape, generator=g).bfloat16().float(),
                           torch.randn(*shape, generator=g).bfloat16().float())
        else:
            cache.state[i] = torch.randn(1, cfg.lin_v_heads, cfg.lin_v_dim, cfg.lin_k_dim, generator=g) * 0.05
            cache.window[i] = torch.randn(1, cfg.conv_kernel - 1, cfg.conv_dim, generator=g).bfloat16().float()
    cache.tokens = (list(prompt_tail) * (ctx // len(prompt_tail) + 1))[:ctx]
    return cache


def _cpu_timed_steps(step_fn, reps: int):
    """One untimed warm-up call of step_fn, then `reps` timed calls. step_fn returns the accepted tokens of
    its step. Returns (median seconds per step, mean accepted tokens per step, per-step seconds)."""
    import statistics

    step_fn()
    secs, toks = [], []
    for _ in range(reps):
        t = time.perf_counter()
        toks.append(step_fn())
        secs.append(time.perf_counter() - t)
    return statistics.median(secs), sum(toks) / len(toks), secs


def _cpu_baseline_e2e(rt, cfg, prompt_tail, args):
    """The oracle's draft-then-verify step on the host cores, over a synthetic 2048-token context: one
    warm-up step, then the median of args.cpu_steps timed steps."""
    import torch

    from oracle import model as OM

    torch.set_num_threads(os.cpu_count() or 1)
    m = OM.CpuHybrid(cfg, rt.w)
    cache = _cpu_cache(cfg, PROMPT_LEN, prompt_tail)
    state = {"t0": int(prompt_tail[-1])}

    def one():
        _, state["t0"], acc = OM.blockspec_step(m, cache, state["t0"], BLOCK, DENOISE)
        return 1 + acc

    med, tok, secs = _cpu_timed_steps(one, max(3, args.cpu_steps))
    return {"value": round(tok / med, 4), "unit": "accepted tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"1 warm-up + {len(secs)} timed draft-then-verify steps (4 denoising passes + verify + greedy "
                      f"acceptance + rollback) of the CPU oracle on the same random-init 4B-shape weights (fp32 "
                      f"arithmetic), synthetic {PROMPT_LEN}-token context; value = mean accepted tokens per step "
                      f"({tok:.2f}) / median step time ({med:.2f} s; steps {[round(x, 2) for x in secs]} s)"}


def _verify_graph_us(step, cache, reps: int = 5) -> float:
    """Median duration of the verify half of a step (verify forward + acceptance + rollback) replayed from
    its own HIP graph, with the cache and t0 restored between replays (outside the events)."""
    import statistics

    import torch

    snap, t0 = cache.snapshot(), step.t0.clone()
    hint = cache.ctx_hint
    cache.ctx_hint = max(hint, cache.Lmax)  # attention splits planned for the capacity (as the step graph)

    def undo():
        cache.restore(snap)
        step.t0.copy_(t0)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step.verify()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    undo()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step.verify()
    torch.cuda.synchronize()
    undo()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3)
        undo()
    cache.ctx_hint = hint
    del g
    return statistics.median(times)


GEOMETRY = ("hidden 2560; 32 layers = 24 gated-delta (16 key / 16 value heads of 128, conv 6144 channels, "
            "kernel 4) + 8 full attention (16 q / 4 kv heads of 256, rotary 64); FFN 9728 SwiGLU; vocab 248320, "
            "tied embedding")


def _forward_roofline(cfg, fwd_us: float, ctx: int, traffic_key: str):
    """HBM roofline of one decoder forward at batch 1: every weight byte once (bf16), the KV cache of the
    8 attention layers and the 24 fp32 GDN states."""
    weight_bytes = cfg.n_params() * 2
    kv_bytes = 8 * 2 * cfg.n_kv_heads * ctx * cfg.head_dim * 2
    state_bytes = 24 * cfg.lin_v_heads * cfg.lin_v_dim * cfg.lin_k_dim * 4
    fwd_bytes = weight_bytes + kv_bytes + state_bytes
    ach = fwd_bytes / (fwd_us * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": "decoder forward (33 canvas rows, every layer)", "achieved": round(ach, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": _measured_traffic(traffic_key), "algorithmic_bytes": fwd_bytes, "avg_us": round(fwd_us, 1)}


def bench_e2e(args, rt=None):
    import torch

    from trida_stack_amd import kernels as K
    from trida_stack_amd.decode import BlockSpecStep
    from trida_stack_amd.model import HybridConfig, build_runtime

    cfg = HybridConfig.four_b()
    rt = rt or build_runtime(cfg, seed=0)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab - 1024, (PROMPT_LEN,), generator=g).tolist()
    total = args.warmup + args.steps
    cache = rt.make_cache(1, max_len=PROMPT_LEN + (BLOCK + 1) * (total + 12) + 64)
    torch.cuda.synchronize()
    t = time.perf_counter()
    logits = rt.prefill(cache, prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t
    step = BlockSpecStep(rt, cache, BLOCK, DENOISE)
    step.t0.fill_(int(logits.argmax()))
    for _ in range(args.warmup):
        step.run()
        cache.ctx_hint += int(step.n_acc[0]) - BLOCK
    torch.cuda.synchronize()
    graph = not args.no_graph
    if graph:
        step.capture()  # the whole step as one HIP graph (the decode loop's default)
    fwd_us = _forward_event_us(rt, cache, step, args) if graph else None
    K.TIMERS, K.TIMER_ONLY = ({}, {"forward", "verify_step"}) if not (args.no_events or graph) else (None, None)
    acc_tokens, hist = 0, [0] * (BLOCK + 1)
    print(f"[bench] e2e bs1: prefill {prefill_s:.2f} s, timing {args.steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(args.steps):
        step.replay() if graph else step.run()
        n = int(step.n_acc[0])  # the host reads the accepted length each step to emit tokens
        cache.ctx_hint += n - BLOCK  # commit counted the whole block; keep the exact length
        acc_tokens += 1 + n
        hist[n] += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t
    timers = K.timer_means_us(K.TIMERS) if K.TIMERS is not None else {}
    if fwd_us is not None:
        timers["forward"] = fwd_us
    K.TIMERS = None
    verify_us = _verify_graph_us(step, cache) if graph else timers.get("verify_step")
    kern = _kernel_breakdown(step, cache, BLOCK, args)
    ctx = int(cache.length[0])
    fwd_us = timers.get("forward")
    roof = _forward_roofline(cfg, fwd_us, ctx, "e2e_forward_bs1") if fwd_us else None
    cpu = None if args.no_cpu else _cpu_baseline_e2e(rt, cfg, prompt[-64:], args)
    value = acc_tokens / elapsed
    return {
        "metric": METRIC, "value": round(value, 2), "unit": "accepted tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random-init weights, random prompt ids)",
        "config": {"workload": "end-to-end self-spec decode, random-init 4B-shape hybrid, batch 1, 2048-token prompt, "
                               "block 32 with 4 denoising passes + verify, greedy acceptance and hybrid rollback",
                   "model_geometry": GEOMETRY, "batch": 1, "prompt_len": PROMPT_LEN, "block": BLOCK,
                   "denoise_passes": DENOISE, "generated_tokens": acc_tokens,
                   "tokens_per_step": round(acc_tokens / args.steps, 3), "accept_hist": hist,
                   "params": cfg.n_params()},
        "verify_step_us": round(verify_us, 1) if verify_us else None,
        "verify_step_how": ("median of 5 HIP-graph replays of the verify half of a step (verify forward + greedy "
                            "acceptance + hybrid rollback), HIP events" if graph else "eager, HIP events"),
        "hip_graph": graph,
        "prefill_s": round(prefill_s, 3),
        "kernel_avg_us": kern,
        "roofline": roof,
        "cpu_baseline": cpu,
        "speedup_vs_cpu": round(value / cpu["value"], 1) if cpu else None,
    }


def bench_generate(rt, n_tokens: int) -> dict:
    """The batch-1 run as the configuration states it: a fresh 2048-token prompt, then draft-then-verify steps
    (4 denoising passes + verify + greedy acceptance + rollback, one HIP-graph replay each, one host read of
    the accepted length per step) until n_tokens are generated; the whole generation is timed, so the
    context grows from 2048 to about 2048 + n_tokens inside the timed region."""
    import torch

    from trida_stack_amd.decode import BlockSpecStep

    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, rt.cfg.vocab - 1024, (PROMPT_LEN,), generator=g).tolist()
    cache = rt.make_cache(1, max_len=PROMPT_LEN + n_tokens + 2 * (BLOCK + 1) + 64)
    logits = rt.prefill(cache, prompt)
    step = BlockSpecStep(rt, cache, BLOCK, DENOISE)
    step.t0.fill_(int(logits.argmax()))
    # one eager step builds the workspaces, then the graph is captured (the decode loop's order); the
    # timed generation starts from the cache that step left
    step.run()
    cache.ctx_hint += int(step.n_acc[0]) - BLOCK
    step.capture()
    torch.cuda.synchronize()
    ctx0 = int(cache.length[0])
    made, steps = 0, 0
    t = time.perf_counter()
    while made < n_tokens:
        step.replay()
        n = int(step.n_acc[0])
        cache.ctx_hint += n - BLOCK
        made += 1 + n
        steps += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t
    return {"value": round(made / elapsed, 2), "unit": "accepted tok/s", "generated_tokens": made, "steps": steps,
            "ms_per_step": round(elapsed * 1e3 / steps, 3), "context": [ctx0, int(cache.length[0])],
            "how": f"{n_tokens} tokens generated after a 2048-token prompt, every step timed (HIP-graph replay, one "
                   "host read per step)"}


def _forward_event_us(rt, cache, step, args, reps: int = 5) -> float:
    """Average duration of one verify forward replayed from its own HIP graph (HIP events on the
    capture stream around the replays), on the live cache: the decoder forward with no launch gaps.
    The forwards only read the cache (a verify pass persists nothing)."""
    import torch

    ids = step.canvas.clone()
    fwd = lambda: rt.forward(ids, cache, "verify")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fwd()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fwd()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    cache.pending = None
    return e0.elapsed_time(e1) * 1e3 / reps


def _kernel_breakdown(step, cache, block, args, steps: int = 4) -> dict:
    """Per-kernel average durations (HIP events around every launch) over a few extra steps after the
    timed region, so the event records do not slow the timed steps."""
    from trida_stack_amd import kernels as K

    if args.no_events:
        return {}
    import torch

    K.TIMERS, K.TIMER_ONLY = {}, None
    for _ in range(steps):
        step.run()
        cache.ctx_hint = max(cache.ctx_hint, int(cache.length.max()))
    torch.cuda.synchronize()
    out = {k: round(v, 2) for k, v in K.timer_means_us(K.TIMERS).items()}
    K.TIMERS = None
    return out


# ------------------------------------------------------------------------------ batch-64 sampled (config 5)
B64, PMIN, PMAX, TEMP, TOP_P = 64, 512, 4096, 0.7, 0.95


def _cpu_baseline_e2e64(rt, cfg, prompts, args):
    """The oracle's sampled draft-then-verify step on the host cores, one sequence of the batch at a time
    (sequences are independent): one warm-up step, then the median of args.cpu_steps timed steps, each for
    another sequence over a synthetic context of its prompt length."""
    import numpy as np
    import torch

    from oracle import model as OM

    torch.set_num_threads(os.cpu_count() or 1)
    m = OM.CpuHybrid(cfg, rt.w)
    rng = np.random.default_rng(0)
    seq = [0]
    lens = []

    def one():
        b = seq[0]
        seq[0] += 1
        cache = _cpu_cache(cfg, len(prompts[b]), prompts[b][-64:], seed=1 + b)
        lens.append(len(prompts[b]))
        _, _, acc = OM.blockspec_sample_step(m, cache, int(prompts[b][-1]), BLOCK, DENOISE, temperature=TEMP,
                                             top_k=0, top_p=TOP_P, rng=rng)
        return 1 + acc

    med, tok, secs = _cpu_timed_steps(one, max(3, args.cpu_steps))
    return {"value": round(tok / med, 4), "unit": "accepted tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"1 warm-up + {len(secs)} timed sampled draft-then-verify steps (4 denoising passes + verify + "
                      f"rejection-sampling acceptance + rollback, temperature {TEMP}, top-p {TOP_P}) of the CPU oracle, "
                      f"one sequence of the batch per step (fp32 arithmetic, float64 sampling), synthetic contexts of "
                      f"the prompt lengths {lens}; the batch of 64 sequences would take 64 such steps; value = mean "
                      f"accepted tokens per sequence step ({tok:.2f}) / median step time ({med:.2f} s; steps "
                      f"{[round(x, 2) for x in secs]} s)"}


def bench_e2e64(args, rt=None):
    import torch

    from trida_stack_amd import kernels as K
    from trida_stack_amd.decode import SamplingParams
    from trida_stack_amd.model import HybridConfig, build_runtime
    from trida_stack_amd.sampling import SampledBlockSpecStep, Sampler, prefill_batch

    cfg = HybridConfig.four_b()
    rt = rt or build_runtime(cfg, seed=0)
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(PMIN, PMAX + 1, (B64,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab - 1024, (n,), generator=g).tolist() for n in lens]
    total = args.warmup + args.steps
    cache = rt.make_cache(B64, max_len=max(lens) + (BLOCK + 1) * (total + 8) + 64)
    smp = Sampler(SamplingParams(temperature=TEMP, top_k=0, top_p=TOP_P, seed=0), rt.dev, ban_id=rt.mask_id)
    torch.cuda.synchronize()
    t = time.perf_counter()
    logits = prefill_batch(rt, cache, prompts)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t
    print(f"[bench] e2e64: prefill of {sum(lens)} prompt tokens in {prefill_s:.1f} s, timing {args.steps} steps",
          file=sys.stderr, flush=True)
    step = SampledBlockSpecStep(rt, cache, BLOCK, DENOISE, smp)
    step.t0.copy_(smp.draw(logits))
    host_len = list(lens)

    def one():
        step.run()
        n = step.n_acc.tolist()  # the host reads the accepted lengths each step to emit tokens
        for b in range(B64):
            host_len[b] += 1 + n[b]
        cache.ctx_hint = max(host_len)
        return n

    for _ in range(args.warmup):
        one()
    torch.cuda.synchronize()
    fwd_us = _forward_event_us(rt, cache, step, args)
    acc_tokens, hist = 0, [0] * (BLOCK + 1)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(args.steps):
        for n in one():
            acc_tokens += 1 + n
            hist[n] += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t
    smp.check()
    step.draw_uniforms()
    verify_us = _verify_graph_us(step, cache, reps=3)
    kern = _kernel_breakdown(step, cache, BLOCK, args, steps=2)
    rows = B64 * (BLOCK + 1)
    ctx_avg = sum(host_len) / B64
    # roofline of the decoder forward at 64 x 33 rows: the GEMMs make it MFMA-bound
    flops = 2 * cfg.n_params() * rows + 8 * 4 * cfg.n_heads * (BLOCK + 1) * ctx_avg * cfg.head_dim * B64
    ach = flops / (fwd_us * 1e-6) / 1e12
    roof = {"bound": "mfma", "kernel": "decoder forward (64 x 33 canvas rows, every layer)",
            "achieved": round(ach, 1), "peak": 2500.0, "unit": "TFLOP/s", "frac": round(ach / 2500.0, 4),
            "traffic": _measured_traffic("e2e_forward_bs64"), "algorithmic_flops": round(flops),
            "avg_us": round(fwd_us, 1)}
    cpu = None if args.no_cpu else _cpu_baseline_e2e64(rt, cfg, prompts, args)
    value = acc_tokens / elapsed
    del step, cache
    return {
        "metric": METRIC, "value": round(value, 2), "unit": "accepted tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random-init weights, random prompt ids)",
        "config": {"workload": "batched sampled self-spec decode, random-init 4B-shape hybrid, batch 64, ragged "
                               "prompts of 512-4096 tokens, block 32 with 4 denoising passes + verify, temperature "
                               "0.7, top-p 0.95, rejection sampling of the causal-head p against the draft q, "
                               "per-sequence KV crops and GDN restores",
                   "model_geometry": GEOMETRY, "batch": B64,
                   "prompt_lens": [min(lens), max(lens), round(sum(lens) / B64, 1)], "block": BLOCK,
                   "denoise_passes": DENOISE, "temperature": TEMP, "top_p": TOP_P,
                   "generated_tokens": acc_tokens, "tokens_per_seq_step": round(acc_tokens / args.steps / B64, 3),
                   "accept_hist": hist, "params": cfg.n_params()},
        "verify_step_us": round(verify_us, 1),
        "verify_step_how": "median of 3 HIP-graph replays of the verify half of a step (verify forward + rejection-"
                           "sampling acceptance + hybrid rollback), HIP events",
        "prefill_s": round(prefill_s, 3),
        "kernel_avg_us": kern,
        "roofline": roof,
        "cpu_baseline": cpu,
        "speedup_vs_cpu": round(value / cpu["value"], 1) if cpu else None,
    }


def bench_canvas(args, rt=None, n: int = 4):
    """The reference's own self-spec algorithm (bd_bidir_shift, decode.py:318-384): one canvas forward of
    2n-1 rows per step, greedy acceptance, the next canvas decided on the device and the rollback, the
    whole step replayed from one HIP graph, batch 1 after a 2048-token prompt. The reference's published
    step time for this algorithm on H100 is 7.5 ms at n = 4 (canvas 7) with vLLM and full CUDA graphs."""
    import statistics

    import torch

    from trida_stack_amd.decode import CanvasSpecStep
    from trida_stack_amd.model import HybridConfig, build_runtime

    cfg = HybridConfig.four_b()
    rt = rt or build_runtime(cfg, seed=0)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab - 1024, (PROMPT_LEN,), generator=g).tolist()
    steps = args.canvas_steps
    cache = rt.make_cache(1, max_len=PROMPT_LEN + n * (steps + 16) + 64)
    logits = rt.prefill(cache, prompt)
    step = CanvasSpecStep(rt, cache, n)
    step.start(logits.argmax().reshape(1))
    step.run()
    step.capture()
    emitted, hist, cold = 0, [0] * n, 0
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(steps):
        step.replay()
        kind, ne = step.kind[:1].tolist()[0], int(step.n_emit[0])  # the host reads the emitted tokens each step
        emitted += ne
        if kind:
            hist[ne - 1] += 1
        else:
            cold += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t
    # one canvas forward, replayed from its own graph
    ids = step.canvas.clone()
    fwd = lambda: rt.forward(ids, cache, "canvas", n_clean=n)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fwd()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        fwd()
    times = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3)
    cache.pending = None
    return {"value": round(emitted / elapsed, 2), "unit": "accepted tok/s", "steps": steps,
            "ms_per_step": round(elapsed * 1e3 / steps, 3), "canvas_forward_us": round(statistics.median(times), 1),
            "tokens_per_step": round(emitted / steps, 3), "accept_hist": hist, "cold_steps": cold,
            "config": {"workload": f"self-spec canvas algorithm (bd_bidir_shift, N = {n}, canvas {2 * n - 1}), "
                                   "batch 1, 2048-token prompt, greedy, one HIP graph per step",
                       "n": n, "canvas": 2 * n - 1},
            "reference_published": "7.5 ms/step on H100 at N = 4 (vLLM, full CUDA graphs, real checkpoint; "
                                   "inference/zoro-1/vllm/docs/SELFSPEC_VLLM_PLAN.md:83)"}


def bench_fwd(args):
    """Decoder forwards only, for counter runs: `steps` eager verify forwards of 33 rows at batch 1 (or
    64 x 33 rows with --fwd-batch 64) over a cache whose committed length is set to 2048 tokens (the
    KV entries and states are zeros; the kernels read them in full all the same), so that every dispatch
    after the weights are drawn belongs to a forward. Prints the per-forward time."""
    import torch

    from trida_stack_amd.model import HybridConfig, build_runtime

    cfg = HybridConfig.four_b()
    rt = build_runtime(cfg, seed=0)
    B = args.fwd_batch
    cache = rt.make_cache(B, max_len=PROMPT_LEN + BLOCK + 1 + 64)
    cache.length.fill_(PROMPT_LEN)
    cache.pos.fill_(PROMPT_LEN)
    cache.tokens = [[0] * PROMPT_LEN for _ in range(B)]
    cache.ctx_hint = PROMPT_LEN
    ids = torch.randint(0, cfg.vocab - 1024, (B, BLOCK + 1), device=rt.dev)
    # a calibration copy of known size (256 MiB read + 256 MiB written), for scaling the counters
    src = torch.ones(64 << 20, dtype=torch.float32, device=rt.dev)
    torch.empty_like(src).copy_(src)
    del src
    for _ in range(max(1, args.warmup)):
        rt.forward(ids, cache, "verify")
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(args.steps):
        rt.forward(ids, cache, "verify")
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t) / args.steps
    return {"workload": f"{args.steps} eager verify forwards, batch {B} x 33 rows, 2048-token context",
            "forwards": args.steps + max(1, args.warmup), "ms_per_forward_eager": round(dt * 1e3, 3)}


def bench_default(args):
    """The headline line: batch 1 (value) and batch 64 (the "bs64" object) on one random-init runtime."""
    import torch

    from trida_stack_amd.model import HybridConfig, build_runtime

    rt = build_runtime(HybridConfig.four_b(), seed=0)
    res = bench_e2e(args, rt)
    sub = argparse.Namespace(**vars(args))
    sub.steps, sub.warmup = args.bs64_steps, args.bs64_warmup
    torch.cuda.empty_cache()
    r64 = bench_e2e64(sub, rt)
    keep = ("value", "unit", "steps", "warmup", "ms_per_step", "verify_step_us", "verify_step_how", "roofline",
            "cpu_baseline", "speedup_vs_cpu", "config", "prefill_s", "kernel_avg_us")
    res["bs64"] = {k: r64[k] for k in keep}
    if args.gen_tokens > 0:
        res[f"gen{args.gen_tokens}"] = bench_generate(rt, args.gen_tokens)
    if args.canvas_steps > 0:
        for n in (4, 8):
            res[f"canvas_n{n}"] = bench_canvas(args, rt, n)
    return res


# ------------------------------------------------------------------------------ chunked GDR (config 2)
def bench_gdr(args):
    """Chunked gated-delta rule of one GDN layer: a 4096-row prefix from a zero state (batch 1, 16 heads,
    d_k = d_v = 128, chunks of 64), a snapshot of the recurrent state [16, 128, 128] fp32 and the conv
    window [3, 8192] bf16, a 32-row verify block on top of the prefix state, and the rollback to a seeded
    accepted length a in [0, 32] (state advanced a rows from the snapshot, window rebuilt)."""
    import torch
    import torch.nn.functional as F

    from trida_stack_amd import kernels as K

    dev = torch.device("cuda:0")
    B, T, H, D, BLK, CH = 1, 4096, 16, 128, 32, 8192
    g0 = torch.Generator(device=dev).manual_seed(0)
    l2 = lambda x: x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    rn = lambda *sh: torch.randn(*sh, generator=g0, device=dev)

    def rows(n):
        return (l2(rn(B, n, H, D)).bfloat16(), l2(rn(B, n, H, D)).bfloat16(), rn(B, n, H, D).bfloat16(),
                (-F.softplus(rn(B, n, H))).contiguous(), torch.sigmoid(rn(B, n, H)).contiguous())

    q, k, v, g, beta = rows(T)
    qb, kb, vb, gb, bb = rows(BLK)
    s0 = torch.zeros(B, H, D, D, device=dev)
    s1, snap = torch.empty_like(s0), torch.empty_like(s0)
    o, ob = torch.empty_like(v), torch.empty_like(vb)
    win, snap_win = rn(B, 3, CH).bfloat16(), torch.empty(B, 3, CH, dtype=torch.bfloat16, device=dev)
    pre = rn(B, BLK, CH).bfloat16()
    a = int(torch.randint(0, BLK + 1, (1,), generator=torch.Generator().manual_seed(0)))
    n_keep = torch.tensor([a], dtype=torch.int32, device=dev)

    prefix = lambda: K.gdr_chunk(q, k, v, g, beta, s0, state_out=s1, out=o)
    snapshot = lambda: K.gdn_snapshot(s1, snap, win, snap_win)
    block = lambda: K.gdr_chunk(qb, kb, vb, gb, bb, s1, causal_mode=1, out=ob)

    def restore():
        K.gdr_chunk(None, kb, vb, gb, bb, snap, state_out=s1, n_keep=n_keep, want_out=False)
        K.gdn_restore(n_keep, snap_window=snap_win, window=win, preconv=pre)

    prefix()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        prefix(), snapshot(), block(), restore()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        prefix(), snapshot(), block(), restore()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    us = {name: _events_time_ms(fn, 50) * 1e3 for name, fn in
          (("prefix", prefix), ("snapshot", snapshot), ("block", block), ("restore", restore))}
    # the token-recurrent kernel over the same prefix, for reference
    rec = lambda: K.gdr_recurrent(q, k, v, g, beta, s0, state_out=s1, out=o)
    us["prefix_token_recurrent"] = _events_time_ms(rec, 3) * 1e3
    C = 64
    flops = (T // C) * H * (C * C * (6 * D + 4 * D) + 6 * C * D * D + 2 * C ** 3 / 3)
    prefix_bytes = 3 * B * T * H * D * 2 + B * T * H * D * 2 + 2 * B * T * H * 4 + 2 * B * H * D * D * 4
    snap_bytes = 2 * (B * H * D * D * 4 + B * 3 * CH * 2)
    total = us["prefix"] + us["snapshot"] + us["block"] + us["restore"]
    tflops = flops / (us["prefix"] * 1e-6) / 1e12
    cpu = None
    if not args.no_cpu:
        from oracle import gdn as OG

        torch.set_num_threads(os.cpu_count() or 1)
        hc = [t.float().cpu() for t in (q, k, v, g, beta)]
        hb = [t.float().cpu() for t in (qb, kb, vb, gb, bb)]
        tt = time.perf_counter()
        _, sT = OG.chunked(*hc, torch.zeros(B, H, D, D))
        snap_h = sT.clone()
        OG.canvas(*hb, sT, num_clean=BLK, causal_mode=1)
        OG.restore(snap_h, win.float().cpu(), *hb[1:], pre.float().cpu(), [a])
        cpu_s = time.perf_counter() - tt
        cpu = {"value": round(cpu_s * 1e6, 1), "unit": "us per prefix + snapshot + block + rollback",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": "one pass of the oracle (torch fp32 on the host): chunked form over the 4096-row prefix, "
                         "snapshot copy, 32-row block, rollback to the same a"}
    return {
        "metric": METRIC, "value": round(total, 2), "unit": "us per prefix (4096 rows) + snapshot + 32-row block + rollback",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 in / fp32 state",
        "data": "synthetic",
        "config": {"workload": "chunked gated-delta rule, batch 1, 16 heads, d_k = d_v = 128, chunk 64, 4096-row "
                               "prefix then 32-row block, snapshot and rollback", "accepted_len": a,
                   "kernel_us": {kk: round(vv, 2) for kk, vv in us.items()},
                   "prefix_gflop": round(flops / 1e9, 3), "prefix_hbm_GBps": round(prefix_bytes / us["prefix"] / 1e3, 1),
                   "snapshot_GBps": round(snap_bytes / us["snapshot"] / 1e3, 1)},
        "roofline": {"bound": "mfma", "kernel": "chunked GDR prefix (gdr_prefix_prep + gdr_prefix_scan)", "achieved": round(tflops, 1),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4),
                     "traffic": _measured_traffic("gdr_prefix_prep", "gdr_prefix_scan")},
        "at_scale": _snapshot_restore_at_scale(dev, H, D, CH),
        "cpu_baseline": cpu,
    }


def _snapshot_restore_at_scale(dev, H, D, CH, L=24, B=64, T=33):
    """Snapshot and rollback over every GDN layer of a batch-64 decode step: L * B state slots
    [H, D, D] fp32 (1.61 GB) and conv windows [3, CH] bf16. The rollback advances each slot from its
    snapshot by that sequence's kept rows (1 + accepted, seeded in [1, T]) and rebuilds the window from
    the block's pre-conv rows; its algorithmic bytes are the state read + write, the kept k / v / g /
    beta rows, the window written and the rows it is rebuilt from."""
    import torch
    import torch.nn.functional as F

    from trida_stack_amd import kernels as K

    NB = L * B
    g = torch.Generator(device=dev).manual_seed(2)
    rn = lambda *sh: torch.randn(*sh, generator=g, device=dev)
    st = rn(NB, H, D, D) * 0.1
    sn = torch.empty_like(st)
    win = rn(NB, 3, CH).bfloat16()
    snw = torch.empty_like(win)
    kb = rn(NB, T, H, D)
    kb = (kb * torch.rsqrt((kb * kb).sum(-1, keepdim=True) + 1e-6)).bfloat16()
    vb = rn(NB, T, H, D).bfloat16()
    gb, bb = (-F.softplus(rn(NB, T, H))).contiguous(), torch.sigmoid(rn(NB, T, H)).contiguous()
    pre = rn(NB, T, CH).bfloat16()
    n_keep = torch.randint(1, T + 1, (B,), generator=g, device=dev, dtype=torch.int32)
    snapshot = lambda: K.gdn_snapshot(st, sn, win, snw)
    restore = lambda: K.gdn_restore(n_keep, snap_state=sn, state=st, k=kb, v=vb, g=gb, beta=bb, snap_window=snw,
                                    window=win, preconv=pre)
    snapshot(), restore()
    torch.cuda.synchronize()
    state_b, win_b = NB * H * D * D * 4, NB * 3 * CH * 2
    kept = int(n_keep.sum()) * L  # kept rows over all slots
    row_b = H * D * 2 * 2 + H * 4 * 2
    snap_bytes = 2 * (state_b + win_b)
    rest_bytes = 2 * state_b + kept * row_b + 2 * win_b
    res = {"workload": f"{L} GDN layers x batch {B}: state [{H}, {D}, {D}] fp32 + window [3, {CH}] bf16 per slot"}
    for name, fn, nb in (("snapshot", snapshot, snap_bytes), ("restore", restore, rest_bytes)):
        us = _events_time_ms(fn, 10) * 1e3
        gbs = nb / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 1), "bytes": nb, "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    # the device's copy ceiling for the same state bytes (torch's copy kernel), and the rollback's state
    # advance in the chunked MFMA form (trida_gdr_chunk with n_keep) against the token-recurrent restore
    us = _events_time_ms(lambda: sn.copy_(st), 10) * 1e3
    res["copy_ceiling"] = {"us": round(us, 1), "bytes": 2 * state_b, "GBps": round(2 * state_b / (us * 1e-6) / 1e9, 1),
                           "kernel": "torch copy_ of the fp32 states"}
    alt = torch.empty_like(st)
    res["restore_state_us"] = {
        "token_recurrent": round(_events_time_ms(lambda: K.gdn_restore(n_keep, snap_state=sn, state=st, k=kb, v=vb, g=gb,
                                                                      beta=bb), 5) * 1e3, 1),
        "chunked_mfma": round(_events_time_ms(lambda: K.gdr_chunk(None, kb, vb, gb, bb, sn, state_out=alt, n_keep=n_keep,
                                                                  want_out=False), 5) * 1e3, 1)}
    del alt
    del st, sn, win, snw, kb, vb, gb, bb, pre
    return res



def bench_gemm(args):
    """The decode-step projection GEMMs (M = 33 rows) of the 4B-shape model: the weight-streaming kernel
    (pre-shuffled weights, the epilogue the forward uses) vs hipBLASLt on the plain weights."""
    import torch

    from trida_stack_amd import kernels as K

    dev = torch.device("cuda:0")
    M = 33
    shapes = {"gate_up": (19456, 2560, K.WS_SILU), "down": (2560, 9728, K.WS_PARTS),
              "gdn_in": (8224, 2560, K.WS_STORE), "attn_qkv": (10240, 2560, K.WS_STORE),
              "gdn_out": (2560, 2048, K.WS_PARTS), "attn_o": (2560, 4096, K.WS_PARTS)}
    calls = {"gate_up": 32, "down": 32, "gdn_in": 24, "attn_qkv": 8, "gdn_out": 24, "attn_o": 8}
    res = {}
    tot_ws = tot_bl = 0.0
    for name, (N, Kd, epi) in shapes.items():
        nbytes = N * Kd * 2
        # enough weight copies (>= 1 GB) that each call streams its weights from HBM, as the layers
        # of a forward do, rather than from the 256 MB last-level cache
        ncopy = max(1, min(16, -(-(1 << 30) // nbytes)))
        x = torch.randn(M, Kd, device=dev).to(torch.bfloat16)
        ws = [(torch.randn(N, Kd, device=dev) * 0.02).to(torch.bfloat16) for _ in range(ncopy)]
        wps = [K.ws_shuffle(w, pair_halves=epi == K.WS_SILU) for w in ws]
        kg = K.ws_plan(N, Kd, epi)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        out = (torch.empty(kg * M * N, dtype=torch.float32, device=dev) if epi == K.WS_PARTS
               else torch.empty(M, N // 2 if epi == K.WS_SILU else N, dtype=torch.bfloat16, device=dev))
        it = itertools.cycle(range(ncopy))
        t_ws = _events_time_ms(lambda: K.ws_gemm(x, wps[next(it)], N, out, epilogue=epi), 48)
        t_bl = _events_time_ms(lambda: torch.matmul(x, ws[next(it)].t(), out=y), 48)
        tot_ws += calls[name] * t_ws * 1e3
        tot_bl += calls[name] * t_bl * 1e3
        res[name] = {"us_ws": round(t_ws * 1e3, 2), "us_hipblaslt": round(t_bl * 1e3, 2), "partial_planes": kg,
                     "GBps_ws": round(nbytes / t_ws / 1e6, 1), "GBps_hipblaslt": round(nbytes / t_bl / 1e6, 1)}
        del ws, wps
    # the row-wise consumer of the partial planes at 33 rows: plain add_rmsnorm (bf16 residual) vs planes
    h = torch.randn(M, 2560, device=dev).to(torch.bfloat16)
    nw = torch.zeros(2560, dtype=torch.bfloat16, device=dev)
    xo = torch.empty_like(h)
    planes = torch.randn(16 * M * 2560, device=dev) * 1e-3
    r = torch.zeros_like(h)
    res["add_rmsnorm_us"] = {"bf16": round(_events_time_ms(lambda: K.add_rmsnorm(h, r, nw, xo), 48) * 1e3, 2)}
    for n in (1, 2, 4, 8, 10, 16):
        res["add_rmsnorm_us"][f"parts{n}"] = round(
            _events_time_ms(lambda: K.add_rmsnorm_parts(h, planes, n, nw, xo), 48) * 1e3, 2)
    big = res["gate_up"]
    ach = big["GBps_ws"]
    return {"metric": METRIC, "value": ach, "unit": "GB/s (gate/up projection + SwiGLU, 33 rows)", "n_gpus": 1,
            "steps": 48, "warmup": 1, "ms_per_step": big["us_ws"] / 1e3, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "decode-step projection GEMMs of the 4B-shape hybrid at 33 rows", "shapes": res,
                       "us_per_forward_ws": round(tot_ws, 1), "us_per_forward_hipblaslt": round(tot_bl, 1)},
            "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None},
            "cpu_baseline": None}


WORKLOADS = {"default": (bench_default, 20, 5), "fwd": (bench_fwd, 8, 1), "canvas": (lambda a: bench_canvas(argparse.Namespace(**dict(vars(a), canvas_steps=a.steps))), 64, 0), "e2e": (bench_e2e, 256, 8), "e2e64": (bench_e2e64, 12, 2), "gdr": (bench_gdr, 20, 3), "accept": (bench_accept, 100, 10), "gemm": (bench_gemm, 50, 1),
             "sample": (bench_sample, 20, 3), "attn": (bench_attn, 100, 10)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="default", choices=sorted(WORKLOADS),
                    help="default: batch 1 (value) plus a batch-64 object; e2e / e2e64: one of them")
    ap.add_argument("--bs64-steps", type=int, default=6, help="default workload: timed batch-64 steps")
    ap.add_argument("--bs64-warmup", type=int, default=2)
    ap.add_argument("--canvas-steps", type=int, default=32, help="default workload: timed canvas-algorithm steps")
    ap.add_argument("--gen-tokens", type=int, default=256, help="default workload: tokens of the timed generation")
    ap.add_argument("--fwd-batch", type=int, default=1, help="fwd workload: sequences per forward")
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--cpu-steps", type=int, default=3, help="timed CPU-oracle steps (median; after one warm-up)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-events", action="store_true", help="skip the live per-kernel event timers")
    ap.add_argument("--no-graph", action="store_true", help="e2e: launch the step eagerly instead of from a HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the step shards by "
              "sequence; see the sharding notes)", file=sys.stderr)
        sys.exit(2)
    fn, steps, warmup = WORKLOADS[args.workload]
    args.steps = steps if args.steps is None else args.steps
    args.warmup = warmup if args.warmup is None else args.warmup
    res = fn(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
