"""The OpenAI-compatible server over the real engine on the GPU: the token ids it serves (plain and
streamed) equal the engine's own greedy self-spec output for the same prompt."""
import http.client
import json
import random
import threading

import pytest

from trida_stack_amd import server as S
from trida_stack_amd.decode import SamplingParams
from trida_stack_amd.engine import Engine
from trida_stack_amd.model import HybridConfig, TridaRuntime, init_weights

pytestmark = pytest.mark.gpu


def post(port, path, body):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=120)
    c.request("POST", path, body=json.dumps(body), headers={"Content-Type": "application/json"})
    r = c.getresponse()
    data = r.read().decode()
    c.close()
    return r.status, data


def test_served_tokens_equal_engine_output(gpu):
    cfg = HybridConfig.tiny()
    rt = TridaRuntime(cfg, init_weights(cfg, seed=0, embed_scale=4.0), device=gpu)
    eng = Engine(rt, mode="self-spec", gen_block=4)
    rng = random.Random(5)
    prompt = [rng.randrange(0, cfg.vocab - 10) for _ in range(23)]
    ref = []
    for ch in eng.generate_ids(prompt, max_tokens=30, sampling=SamplingParams(temperature=0.0)):
        ref.extend(ch)
    st = S.ServerState(eng, None, model_name="random-tiny")
    srv = S.make_server(st, "127.0.0.1", 0)
    threading.Thread(target=srv.serve_forever, daemon=True).start()
    try:
        port = srv.server_address[1]
        code, data = post(port, "/v1/completions", {"prompt": prompt, "max_tokens": 30, "temperature": 0})
        assert code == 200, data
        r = json.loads(data)
        assert r["choices"][0]["token_ids"] == ref
        assert r["usage"]["completion_tokens"] == len(ref) and r["usage"]["trida"]["forwards"] > 0
        code, data = post(port, "/v1/completions", {"prompt": prompt, "max_tokens": 30, "stream": True, "temperature": 0})
        ids = []
        for block in data.split("\n\n"):
            if block.startswith("data: {"):
                ids.extend(json.loads(block[6:])["choices"][0].get("token_ids", []))
        assert code == 200 and ids == ref
        code, data = post(port, "/v1/completions", {"prompt": prompt, "max_tokens": 30, "mode": "causal", "temperature": 0})
        assert code == 200 and json.loads(data)["choices"][0]["token_ids"] == ref  # greedy AR == greedy self-spec
    finally:
        srv.shutdown()
        srv.server_close()
