"""OpenAI-compatible server (trida_stack_amd.server) on the CPU: routes, request checks, stop strings,
server-sent-event streaming and usage, driven by a scripted engine and a character tokenizer so that
only the server's own logic is under test."""
import http.client
import json

import pytest

from trida_stack_amd import server as S
from trida_stack_amd.decode import DecodeStats


class CharTokenizer:
    """Token i is chr(i): encode / decode are exact, one token per character."""

    chat_template = None

    def encode(self, text):
        return [ord(c) for c in text]

    def decode(self, ids):
        return "".join(chr(i) for i in ids)


class ScriptedEngine:
    """generate_ids yields the script in chunks (as self-spec does) and fills the stats."""

    class rt:
        class cfg:
            vocab = 1 << 16

    def __init__(self, script, chunk=3, eos=False):
        self.script, self.chunk, self.eos = script, chunk, eos
        self.calls = []

    def generate_ids(self, prompt, *, max_tokens, sampling=None, mode=None, stats=None):
        self.calls.append({"prompt": list(prompt), "max_tokens": max_tokens, "sampling": sampling, "mode": mode})
        stats.prompt_tokens = len(prompt)
        out = self.script[:max_tokens]
        for i in range(0, len(out), self.chunk):
            stats.new_tokens += len(out[i:i + self.chunk])
            stats.forwards += 1
            yield out[i:i + self.chunk]
        stats.finish_reason = "stop" if self.eos and len(self.script) <= max_tokens else "length"


@pytest.fixture
def serve():
    servers = []

    def start(engine, tokenizer=CharTokenizer(), **defaults):
        st = S.ServerState(engine, tokenizer, model_name="tiny", defaults=defaults or None)
        srv = S.make_server(st, "127.0.0.1", 0)
        import threading

        threading.Thread(target=srv.serve_forever, daemon=True).start()
        servers.append(srv)
        return srv.server_address[1]

    yield start
    for srv in servers:
        srv.shutdown()
        srv.server_close()


def request(port, method, path, body=None):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=30)
    c.request(method, path, body=None if body is None else json.dumps(body),
              headers={"Content-Type": "application/json"})
    r = c.getresponse()
    data = r.read().decode()
    c.close()
    return r.status, data


def test_models_health_and_unknown_routes(serve):
    port = serve(ScriptedEngine([1]))
    code, data = request(port, "GET", "/v1/models")
    assert code == 200 and json.loads(data)["data"][0]["id"] == "tiny"
    assert request(port, "GET", "/health")[0] == 200
    assert request(port, "GET", "/nope")[0] == 404
    assert request(port, "POST", "/v1/nope", {})[0] == 404


def test_completion_text_usage_and_sampling_fields(serve):
    eng = ScriptedEngine([ord(c) for c in "hello world"], eos=True)
    port = serve(eng)
    code, data = request(port, "POST", "/v1/completions",
                         {"prompt": "say hi", "max_tokens": 64, "temperature": 0.7, "top_p": 0.9, "top_k": 20,
                          "seed": 3})
    assert code == 200, data
    r = json.loads(data)
    assert r["object"] == "text_completion" and r["choices"][0]["text"] == "hello world"
    assert r["choices"][0]["finish_reason"] == "stop"
    assert r["usage"]["prompt_tokens"] == 6 and r["usage"]["completion_tokens"] == 11
    assert r["usage"]["total_tokens"] == 17 and "trida" in r["usage"]
    sp = eng.calls[0]["sampling"]
    assert (sp.temperature, sp.top_p, sp.top_k, sp.seed) == (0.7, 0.9, 20, 3)
    assert eng.calls[0]["prompt"] == [ord(c) for c in "say hi"]


def test_budget_and_context_length(serve):
    eng = ScriptedEngine(list(range(65, 91)))
    port = serve(eng, context_length=16)
    code, data = request(port, "POST", "/v1/completions", {"prompt": "abcdef", "max_tokens": 100})
    assert code == 200 and eng.calls[-1]["max_tokens"] == 10  # capped at context - prompt
    assert json.loads(data)["choices"][0]["finish_reason"] == "length"
    code, data = request(port, "POST", "/v1/completions", {"prompt": "x" * 16})
    err = json.loads(data)["error"]
    assert code == 400 and err["code"] == "context_length_exceeded"
    request(port, "POST", "/v1/completions", {"prompt": "ab", "max_tokens": -5})
    assert eng.calls[-1]["max_tokens"] == 1  # at least one token, as the reference server clamps
    assert request(port, "POST", "/v1/completions", {"prompt": "ab", "max_tokens": "many"})[0] == 400


def test_stop_strings_cut_the_text(serve):
    port = serve(ScriptedEngine([ord(c) for c in "one. two. three."]))
    code, data = request(port, "POST", "/v1/completions", {"prompt": "go", "stop": [" two", "zzz"]})
    r = json.loads(data)
    assert code == 200 and r["choices"][0]["text"] == "one." and r["choices"][0]["finish_reason"] == "stop"


def test_token_id_prompts_without_tokenizer(serve):
    eng = ScriptedEngine([5, 6, 7, 8])
    port = serve(eng, tokenizer=None)
    code, data = request(port, "POST", "/v1/completions", {"prompt": [1, 2, 3], "max_tokens": 3})
    r = json.loads(data)
    assert code == 200 and r["choices"][0]["token_ids"] == [5, 6, 7] and r["choices"][0]["text"] == ""
    assert request(port, "POST", "/v1/completions", {"prompt": "text"})[0] == 400  # no tokenizer
    assert request(port, "POST", "/v1/completions", {"prompt": [1, -2]})[0] == 400  # out of range ids
    assert request(port, "POST", "/v1/completions", {"prompt": [1, 1 << 16]})[0] == 400
    assert request(port, "POST", "/v1/chat/completions", {"messages": [{"role": "user", "content": "x"}]})[0] == 400


def test_chat_completion_without_template(serve):
    eng = ScriptedEngine([ord(c) for c in "fine"], eos=True)
    port = serve(eng)
    code, data = request(port, "POST", "/v1/chat/completions",
                         {"messages": [{"role": "system", "content": "be brief"},
                                       {"role": "user", "content": [{"type": "text", "text": "how are you"}]}]})
    r = json.loads(data)
    assert code == 200 and r["object"] == "chat.completion"
    assert r["choices"][0]["message"] == {"role": "assistant", "content": "fine"}
    assert eng.calls[0]["prompt"] == [ord(c) for c in "system: be brief\nuser: how are you\nassistant:"]


def sse_events(data):
    out = []
    for block in data.split("\n\n"):
        if block.startswith("data: "):
            p = block[len("data: "):]
            out.append(p if p == "[DONE]" else json.loads(p))
    return out


def test_streaming_chat_and_completion(serve):
    port = serve(ScriptedEngine([ord(c) for c in "streamed text"], chunk=4, eos=True))
    code, data = request(port, "POST", "/v1/chat/completions",
                         {"messages": [{"role": "user", "content": "hi"}], "stream": True,
                          "stream_options": {"include_usage": True}})
    ev = sse_events(data)
    assert code == 200 and ev[-1] == "[DONE]"
    assert ev[0]["choices"][0]["delta"] == {"role": "assistant"}
    assert "".join(e["choices"][0]["delta"].get("content", "") for e in ev[1:-2] if e["choices"]) == "streamed text"
    assert ev[-3]["choices"][0]["finish_reason"] == "stop"
    assert ev[-2]["usage"]["completion_tokens"] == 13
    code, data = request(port, "POST", "/v1/completions", {"prompt": "x", "stream": True, "max_tokens": 6})
    ev = sse_events(data)
    assert "".join(e["choices"][0]["text"] for e in ev[:-1]) == "stream"
    assert ev[-2]["choices"][0]["finish_reason"] == "length"


def test_bad_requests(serve):
    port = serve(ScriptedEngine([1]))
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=30)
    c.request("POST", "/v1/completions", body="{not json", headers={"Content-Type": "application/json"})
    assert c.getresponse().status == 400
    c.close()
    assert request(port, "POST", "/v1/completions", {"prompt": "a", "temperature": "hot"})[0] == 400
    assert request(port, "POST", "/v1/completions", {"prompt": "a", "stop": [1]})[0] == 400
    assert request(port, "POST", "/v1/completions", {"prompt": "a", "mode": "warp"})[0] == 400
    assert request(port, "POST", "/v1/chat/completions", {"messages": []})[0] == 400


def test_engine_errors_are_reported(serve):
    class Failing(ScriptedEngine):
        def generate_ids(self, prompt, **kw):
            raise ValueError("diffusion mode decodes greedily (temperature 0)")
            yield []

    port = serve(Failing([1]))
    code, data = request(port, "POST", "/v1/completions", {"prompt": "a", "mode": "diffusion", "temperature": 1})
    assert code == 400 and "greedily" in json.loads(data)["error"]["message"]
