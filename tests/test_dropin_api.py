"""CPU: the Python drop-in surface keeps the reference's names, keywords, defaults and decode-config
keys (inference/zoro-1/mlx/trida_mlx/engine.py, decode.py; inference/zoro-1/configs/*.yaml), and the
host-side logic behind them (loop guard, prompt-cache slots, decode configs) behaves like the
reference's. No GPU: the engine's cache logic runs on a stub runtime."""
import inspect

import pytest
import torch

from trida_stack_amd import decode as D
from trida_stack_amd import decode_config as DC
from trida_stack_amd import engine as E
from trida_stack_amd.model import HybridConfig, TridaRuntime, init_weights


def test_engine_keywords_match_reference():
    # Engine.__init__(model, *, mode, gen_block, prefill_chunk, prompt_cache, fused_gdn, cache_slots, ...)
    # (engine.py:60-62) and generate_ids(prompt, *, max_tokens, sampling, mode, stats, progress, stop_ids)
    # (engine.py:228-230)
    init = inspect.signature(E.Engine.__init__).parameters
    for k in ("model", "mode", "gen_block", "prefill_chunk", "prompt_cache", "fused_gdn", "cache_slots"):
        assert k in init, k
    assert init["prefill_chunk"].default == 512 and init["prompt_cache"].default is True
    assert init["cache_slots"].default == 3 and init["mode"].default == "self-spec"
    gen = inspect.signature(E.Engine.generate_ids).parameters
    for k in ("prompt", "max_tokens", "sampling", "mode", "stats", "progress", "stop_ids"):
        assert k in gen, k
    assert gen["max_tokens"].default == 2048
    for name in ("reset_cache", "cached_tokens", "render", "encode", "generate_text", "warmup"):
        assert callable(getattr(E.Engine, name))


def test_sampling_params_defaults_and_fields():
    sp = D.SamplingParams()
    assert (sp.temperature, sp.top_k, sp.top_p, sp.seed) == (1.0, 50, 0.95, None)  # decode.py:36-40
    assert sp.banned == () and sp.gate == () and sp.gate_log is None
    assert not sp.greedy and D.SamplingParams(temperature=0.0).greedy
    assert D.GATE_NOTE_MIN == 0.05
    st = D.DecodeStats()
    assert st.gate_blocked == [] and st.loop_stopped_thinking is False
    d = st.as_dict()
    assert "gate_blocked" not in d and "loop_stopped_thinking" not in d
    st.gate_blocked, st.loop_stopped_thinking = [0.3], True
    d = st.as_dict()
    assert d["gate_blocked"] == [0.3] and d["loop_stopped_thinking"] is True


def test_looping_detects_repeated_blocks():
    assert D.looping(list(range(200))) == 0
    hist = [7, 8, 9] + [1, 2, 3, 4] * 30          # period 4, 120 tokens of repeats
    assert D.looping(hist) == 4
    assert D.looping([1, 2, 3, 4] * 5) == 0          # 20 tokens: below the 96-token span
    assert D.looping([5] * 95) == 0 and D.looping([5] * 96) == 1
    p = 20
    block = list(range(100, 100 + p))
    assert D.looping([0] * 3 + block * 6) == p        # 6 repeats of 20 = 120 >= 96
    assert D.looping([0] * 3 + block * 5) == 0        # 5 repeats fall short


def _looping_brute(hist: list) -> int:
    """decode.py:178-195 as written there: the tail compared with itself shifted, for each p in turn."""
    n = len(hist)
    for p in range(1, min(D.LOOP_MAX_PERIOD, n // D.LOOP_MIN_REPEATS) + 1):
        span = max(p * D.LOOP_MIN_REPEATS, D.LOOP_MIN_SPAN)
        if span > n:
            break
        tail = hist[n - span:]
        if tail[p:] == tail[:-p]:
            return p
    return 0


def test_looping_matches_shifted_tail_rule():
    """The Z-array form answers exactly the shifted-tail comparison of every period."""
    import random

    rng = random.Random(7)
    for _ in range(400):
        p = rng.choice([1, 2, 3, 5, 16, 17, 64, 200, 256, 257])
        block = [rng.randrange(3) for _ in range(p)]
        hist = [rng.randrange(3) for _ in range(rng.randrange(40))] + block * rng.randrange(9)
        hist += [rng.randrange(3) for _ in range(rng.randrange(3))]
        assert D.looping(hist) == _looping_brute(hist)


class _ByteTok:
    """A byte-level tokenizer: id = one UTF-8 byte."""

    def decode(self, ids, skip_special_tokens=False):
        return bytes(ids).decode("utf-8", errors="replace")


def test_incremental_detokenizer_streams_exact_text():
    """The deltas concatenate to the full decode, and never end inside a multi-byte character."""
    import random

    text = "plain ascii, ünïcödé, 漢字かな, emoji 🙂🚀 and more text " * 3
    ids = list(text.encode("utf-8"))
    rng = random.Random(3)
    for _ in range(20):
        det = E.IncrementalDetokenizer(_ByteTok())
        out, i = [], 0
        while i < len(ids):
            k = rng.randrange(1, 6)
            piece = det.add(ids[i: i + k])
            assert "\ufffd" not in piece
            out.append(piece)
            i += k
        assert "".join(out) == text


def test_ngram_loop_window():
    ng = D.NgramLoop(n=4, window=40, frac=0.5)
    hist = []
    fired = None
    for i in range(200):
        hist.append(i % 10)                         # period 10: every 4-gram recurs after 10 tokens
        if ng.add(hist) and fired is None:
            fired = i
    assert fired == 3 + 40 - 1  # the first time the window holds 40 phrases (30 of them repeats)
    ng2 = D.NgramLoop(n=4, window=40, frac=0.5)
    hist = []
    assert not any(ng2.add(hist) for hist in ([*range(k)] for k in range(1, 120)))


def test_emitter_loop_guard():
    st = D.DecodeStats()
    em = D._Emitter(st, 10_000, set())
    assert D._Emitter.loop_guard is False
    out = []
    for _ in range(100):
        out += em([1, 2, 3])
    assert not em.done and st.finish_reason == "length"  # off by default
    try:
        D._Emitter.loop_guard = True
        st = D.DecodeStats()
        em = D._Emitter(st, 10_000, set())
        n = 0
        while not em.done and n < 1000:
            n += len(em([1, 2, 3]))
        assert em.done and st.finish_reason == "repetition" and n < 200
    finally:
        D._Emitter.loop_guard = False
    st = D.DecodeStats()
    em = D._Emitter(st, 5, {9})
    assert em([1, 2, 9, 4]) == [1, 2] and st.finish_reason == "stop" and st.stop_token == 9


def test_decode_config_keys():
    # the reference's self-spec config (inference/zoro-1/configs/zoro1_self_spec_b15_g8.yaml:3-12)
    ref = {"variant": "bd_bidir_shift", "block_size": 15, "gen_block_size": 8, "mask_id": 248077,
           "causal_prefill": True, "temperature": 1.0, "top_k": 20, "top_p": 0.95, "use_spec_verify": True,
           "draft_mode": "strict_truncated"}
    cfg = DC.parse(ref)
    assert cfg.engine_kwargs() == {"gen_block": 8}
    sp = cfg.sampling()
    assert (sp.temperature, sp.top_k, sp.top_p) == (1.0, 20, 0.95)
    packaged = DC.for_mode("self-spec")
    assert packaged == cfg and DC.for_mode("causal") is None
    with pytest.raises(ValueError, match="block_size"):
        DC.parse(dict(ref, block_size=16))
    with pytest.raises(ValueError, match="variant"):
        DC.parse(dict(ref, variant="low_confidence"))
    with pytest.raises(ValueError, match="unknown"):
        DC.parse(dict(ref, bogus=1))
    with pytest.raises(ValueError, match="mask_id"):
        cfg.check_mask(5)
    assert DC.parse({"threshold": 0.8}).engine_kwargs() == {"threshold": 0.8}


class _StubCache:
    """The SeqCache surface the engine's prompt cache touches."""

    def __init__(self, max_len):
        self.tokens = [[]]
        self.Lmax = max_len

    def snapshot(self):
        return (None, None, None, None, [list(self.tokens[0])])

    def restore(self, snap):
        self.tokens = [list(snap[4][0])]


class _StubRuntime(TridaRuntime):
    def __init__(self):
        cfg = HybridConfig.tiny()
        super().__init__(cfg, {}, device="cpu")
        self.prefills = []

    def make_cache(self, batch=1, max_len=4096):
        return _StubCache(max_len)

    def prefill(self, cache, tokens, seq=0):
        self.prefills.append(list(tokens))
        cache.tokens[seq].extend(tokens)
        if self.progress_cb is not None:
            self.progress_cb(len(tokens))
        return torch.zeros(self.cfg.vocab)


class _Tok:
    unk_token_id = -1

    def convert_tokens_to_ids(self, t):
        return {"<|im_start|>": 100}.get(t, -1)


def test_prompt_cache_slots_and_snapshots():
    """engine.py:146-198: a prompt resumes from the longest proper-prefix live cache or snapshot; the
    system block and the last <|im_start|> are snapshotted; slots are reused LRU."""
    eng = E.Engine(_StubRuntime(), tokenizer=_Tok(), cache_slots=2)
    assert eng.im_start == 100 and eng.cached_tokens() == [0]
    sys_blk = [100, 1, 2, 3]
    turn1 = sys_blk + [100, 10, 11, 100, 12]
    eng._position_cache(turn1)
    eng._prefill_to_snapshot(turn1)
    assert set(eng.cur.snaps) == {"system", "last"}
    assert eng.cache.tokens[0] == turn1[:7]  # prefilled up to the last <|im_start|>
    eng.rt.prefill(eng.cache, turn1[7:] + [50, 51])  # the generation commits its reply
    slot1 = eng.cur
    # the next turn re-renders the history: it extends the live tokens, so they are reused
    turn2 = turn1 + [50, 51, 100, 13, 100, 14]
    eng._position_cache(turn2)
    assert eng.cur is slot1 and len(eng.cache.tokens[0]) == len(turn1) + 2
    # a rewritten history that keeps only the system block resumes from its snapshot
    other = sys_blk + [100, 99, 98]
    eng._position_cache(other)
    assert eng.cur is slot1 and eng.cache.tokens[0] == sys_blk
    assert "last" not in eng.cur.snaps  # no longer a prefix of what the cache holds
    # an unrelated prompt takes a second slot, then the least recently used one
    eng._position_cache([7, 7, 7])
    assert eng.cur is not slot1 and len(eng.slots) == 2 and eng.cache.tokens[0] == []
    eng.rt.prefill(eng.cache, [7, 7])
    eng._position_cache([8, 8, 8])
    assert len(eng.slots) == 2 and eng.cur is slot1 and eng.cache.tokens[0] == []
    # prompt_cache=False: a fresh cache every time
    eng2 = E.Engine(_StubRuntime(), tokenizer=_Tok(), prompt_cache=False)
    eng2._position_cache(turn1)
    eng2._prefill_to_snapshot(turn1)
    assert eng2.cur.snaps == {} and eng2.cache.tokens[0] == []


def test_engine_keywords_reach_runtime():
    rt = _StubRuntime()
    eng = E.Engine(rt, prefill_chunk=128, fused_gdn=True, gen_block=8)
    assert rt.prefill_chunk == 128 and rt.fused_gdn is True and eng.n == 8
    assert E.Engine(_StubRuntime(), fused_gdn=None).rt.fused_gdn is False


def test_cli_reads_decode_config(tmp_path):
    from trida_stack_amd import cli

    p = tmp_path / "c.yaml"
    p.write_text("variant: bd_bidir_shift\nblock_size: 7\ngen_block_size: 5\n")
    with pytest.raises(SystemExit):
        cli.main(["--config", str(p), "--mode", "decide"])
    with pytest.raises(ValueError, match="block_size"):
        cli.main(["--config", str(p)])
