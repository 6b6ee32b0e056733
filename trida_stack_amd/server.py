"""OpenAI-compatible HTTP server over the Engine: the surface of the reference's server
(inference/zoro-1/mlx/trida_mlx/server.py:383-439): ``GET /v1/models``, ``/health``; ``POST
/v1/completions`` and ``/v1/chat/completions``, streamed as server-sent events when ``"stream": true``.

One worker thread owns the engine, and so the GPU. Request threads queue jobs to it and read their
deltas back, as the reference's worker and job classes do (server.py:176-345). A client that
disconnects cancels its job between decode steps. Sampling fields follow the reference's
``_sampling`` (server.py:41-52): temperature, top_k, top_p, seed. The budget is max_tokens (or
max_completion_tokens) capped by the context length (server.py:459-466). Usage reports the decode
stats under ``"trida"`` (server.py:506-510).

The reference server's decision head, vision inputs, tool-call parsing and the systemone / decide routes
are not part of the decode path and are not served.

    python -m trida_stack_amd.server --model CHECKPOINT_DIR [--mode self-spec] [--port 8000]
"""
from __future__ import annotations

import argparse
import json
import queue
import threading
import time
import uuid
from http.server import BaseHTTPRequestHandler, ThreadingHTTPServer
from typing import Callable, Optional

from .decode import DecodeStats, SamplingParams

DEFAULTS = {"temperature": 1.0, "top_k": 50, "top_p": 0.95, "max_tokens": 512, "context_length": 32768}


class BadRequest(ValueError):
    """A request the server rejects with HTTP 400."""

    def __init__(self, msg: str, code: Optional[str] = None, param: Optional[str] = None):
        super().__init__(msg)
        self.code, self.param = code, param


def sampling_of(body: dict, defaults: dict) -> SamplingParams:
    t = body.get("temperature", defaults["temperature"])
    try:
        return SamplingParams(temperature=float(t if t is not None else defaults["temperature"]),
                              top_k=int(body.get("top_k") or defaults["top_k"]),
                              top_p=float(body.get("top_p") or defaults["top_p"]),
                              seed=body.get("seed"))
    except (TypeError, ValueError) as e:
        raise BadRequest(f"sampling parameters: {e}")


def budget(prompt: list, body: dict, defaults: dict) -> int:
    ctx = defaults["context_length"]
    if len(prompt) >= ctx:
        raise BadRequest(f"This model's maximum context length is {ctx} tokens. However, your messages resulted in "
                         f"{len(prompt)} tokens. Please reduce the length of the messages.",
                         code="context_length_exceeded", param="messages")
    want = body.get("max_completion_tokens") or body.get("max_tokens") or defaults["max_tokens"]
    try:
        want = int(want)
    except (TypeError, ValueError):
        raise BadRequest("max_tokens must be an integer")
    return max(1, min(want, ctx - len(prompt)))


def stops_of(body: dict) -> list:
    s = body.get("stop")
    s = [s] if isinstance(s, str) else (s or [])
    if not all(isinstance(x, str) for x in s):
        raise BadRequest("stop must be a string or a list of strings")
    return [x for x in s if x]


class Job:
    """One generation: runs on the worker thread and posts ("delta", text, ids), then ("done", text,
    ids, stats, finish_reason) or ("error", exception) to its queue."""

    def __init__(self, prompt: list, sampling: SamplingParams, max_tokens: int, stops: list, mode: Optional[str]):
        self.prompt, self.sampling, self.max_tokens, self.stops, self.mode = prompt, sampling, max_tokens, stops, mode
        self.out: queue.Queue = queue.Queue()
        self.cancelled = False

    def run(self, engine, tokenizer) -> None:
        stats = DecodeStats()
        ids: list = []
        text, sent = "", 0
        finish = None
        gen = engine.generate_ids(self.prompt, max_tokens=self.max_tokens, sampling=self.sampling, mode=self.mode,
                                  stats=stats)
        try:
            for chunk in gen:
                if self.cancelled:
                    break
                ids.extend(chunk)
                if tokenizer is None:
                    self.out.put(("delta", "", list(chunk)))
                    continue
                text = tokenizer.decode(ids)
                cut = min((i for i in (text.find(s) for s in self.stops) if i >= 0), default=-1)
                if cut >= 0:
                    text, finish = text[:cut], "stop"
                # hold back a trailing partial character until the next chunk completes it
                end = len(text) if finish or not text.endswith("\ufffd") else len(text.rstrip("\ufffd"))
                if end > sent:
                    self.out.put(("delta", text[sent:end], list(chunk)))
                    sent = end
                if finish:
                    break
        finally:
            gen.close()
        if tokenizer is not None and sent < len(text):
            self.out.put(("delta", text[sent:], []))
        if finish is None:
            # the loop guard's cut ("repetition") is reported as a cut reply, "length" (server.py:554-555)
            finish = "stop" if stats.finish_reason == "stop" else "length"
        self.out.put(("done", text, ids, stats, finish))


class Worker(threading.Thread):
    """The only thread that calls the engine."""

    def __init__(self, engine, tokenizer):
        super().__init__(daemon=True, name="trida-engine")
        self.engine, self.tokenizer = engine, tokenizer
        self.jobs: queue.Queue = queue.Queue()

    def submit(self, job: Job) -> None:
        self.jobs.put(job)

    def run(self) -> None:
        while True:
            job = self.jobs.get()
            if job is None:
                return
            if job.cancelled:
                continue
            try:
                job.run(self.engine, self.tokenizer)
            except Exception as e:  # noqa: BLE001 - reported to the request thread
                job.out.put(("error", e))


class ServerState:
    def __init__(self, engine, tokenizer=None, model_name: str = "trida", defaults: Optional[dict] = None):
        self.engine, self.tokenizer, self.model_name = engine, tokenizer, model_name
        self.defaults = dict(DEFAULTS, **(defaults or {}))
        cfg = getattr(getattr(engine, "rt", None), "cfg", None)
        self.vocab = getattr(cfg, "vocab", None)  # token ids are checked against it before they reach the GPU
        self.worker = Worker(engine, tokenizer)
        self.worker.start()
        self.created = int(time.time())

    # ---- prompts
    def completion_prompt(self, body: dict) -> list:
        p = body.get("prompt")
        if isinstance(p, list) and p and all(isinstance(t, int) and not isinstance(t, bool) for t in p):
            if self.vocab is not None and not all(0 <= t < self.vocab for t in p):
                raise BadRequest(f"token ids must lie in [0, {self.vocab})", param="prompt")
            return list(p)
        if isinstance(p, list) and len(p) == 1 and isinstance(p[0], (str, list)):
            return self.completion_prompt(dict(body, prompt=p[0]))
        if isinstance(p, str):
            if self.tokenizer is None:
                raise BadRequest("this model has no tokenizer: send the prompt as a list of token ids")
            return list(self.tokenizer.encode(p))
        raise BadRequest("prompt must be a string or a list of token ids (one prompt per request)", param="prompt")

    def chat_prompt(self, body: dict) -> list:
        msgs = body.get("messages")
        if not isinstance(msgs, list) or not msgs:
            raise BadRequest("messages must be a non-empty list", param="messages")
        norm = []
        for m in msgs:
            if not isinstance(m, dict) or "role" not in m:
                raise BadRequest("every message needs a role", param="messages")
            c = m.get("content") or ""
            if isinstance(c, list):  # content parts: the text ones
                c = "".join(part.get("text", "") for part in c if isinstance(part, dict) and part.get("type") == "text")
            norm.append({"role": str(m["role"]), "content": str(c)})
        if self.tokenizer is None:
            raise BadRequest("this model has no tokenizer: use /v1/completions with token ids")
        if getattr(self.tokenizer, "chat_template", None):
            ids = self.tokenizer.apply_chat_template(norm, add_generation_prompt=True, tokenize=True)
            return list(ids["input_ids"] if isinstance(ids, dict) else ids)
        text = "".join(f"{m['role']}: {m['content']}\n" for m in norm) + "assistant:"
        return list(self.tokenizer.encode(text))

    def usage(self, stats: DecodeStats) -> dict:
        return {"prompt_tokens": stats.prompt_tokens, "completion_tokens": stats.new_tokens,
                "total_tokens": stats.prompt_tokens + stats.new_tokens,
                "prompt_tokens_details": {"cached_tokens": stats.reused_tokens}, "trida": stats.as_dict()}

    def generate(self, prompt: list, body: dict, on_delta: Callable[[str, list], None]):
        """Queues a job and relays its deltas; returns (text, ids, stats, finish_reason). Any exception
        raised by on_delta (a closed connection) cancels the job."""
        mode = body.get("mode")
        if mode is not None and mode not in ("causal", "self-spec", "diffusion"):
            raise BadRequest("mode must be causal, self-spec or diffusion", param="mode")
        sp = sampling_of(body, self.defaults)
        if (mode or getattr(self.engine, "mode", None)) == "diffusion" and body.get("temperature") is None:
            sp.temperature = 0.0  # block diffusion decodes greedily
        job = Job(prompt, sp, budget(prompt, body, self.defaults), stops_of(body), mode)
        self.worker.submit(job)
        try:
            while True:
                kind, *val = job.out.get()
                if kind == "delta":
                    on_delta(val[0], val[1])
                elif kind == "error":
                    e = val[0]
                    raise BadRequest(str(e)) if isinstance(e, ValueError) else e
                else:
                    return tuple(val)
        except BaseException:
            job.cancelled = True
            raise


def make_handler(state: ServerState):
    class Handler(BaseHTTPRequestHandler):
        protocol_version = "HTTP/1.1"

        def log_message(self, fmt, *args):  # quiet
            pass

        def _json(self, code: int, obj: dict) -> None:
            data = json.dumps(obj).encode()
            self.send_response(code)
            self.send_header("Content-Type", "application/json")
            self.send_header("Content-Length", str(len(data)))
            self.send_header("Access-Control-Allow-Origin", "*")
            self.end_headers()
            self.wfile.write(data)

        def _sse_start(self) -> None:
            self.send_response(200)
            self.send_header("Content-Type", "text/event-stream")
            self.send_header("Cache-Control", "no-cache")
            self.send_header("Connection", "close")
            self.send_header("Access-Control-Allow-Origin", "*")
            self.end_headers()
            self.close_connection = True

        def _sse(self, obj) -> None:
            payload = obj if isinstance(obj, str) else json.dumps(obj)
            self.wfile.write(f"data: {payload}\n\n".encode())
            self.wfile.flush()

        def do_OPTIONS(self):
            self.send_response(204)
            self.send_header("Access-Control-Allow-Origin", "*")
            self.send_header("Access-Control-Allow-Methods", "GET, POST, OPTIONS")
            self.send_header("Access-Control-Allow-Headers", "*")
            self.send_header("Content-Length", "0")
            self.end_headers()

        def _card(self) -> dict:
            return {"id": state.model_name, "object": "model", "created": state.created, "owned_by": "trida",
                    "context_length": state.defaults["context_length"]}

        def do_GET(self):
            path = self.path.split("?")[0].rstrip("/")
            if path in ("/v1/models", "/models"):
                return self._json(200, {"object": "list", "data": [self._card()]})
            if path in ("/v1/models/" + state.model_name, "/models/" + state.model_name):
                return self._json(200, self._card())
            if path in ("/health", "/v1/health", ""):
                return self._json(200, {"status": "ok", "model": state.model_name})
            self._json(404, {"error": {"message": f"no route {self.path}"}})

        def do_POST(self):
            route = self.path.split("?")[0].rstrip("/")
            try:
                n = int(self.headers.get("Content-Length") or 0)
                try:
                    body = json.loads(self.rfile.read(n) or b"{}")
                except json.JSONDecodeError as e:
                    raise BadRequest(f"invalid JSON: {e}")
                if not isinstance(body, dict):
                    raise BadRequest("the request body must be a JSON object")
                if route in ("/v1/chat/completions", "/chat/completions"):
                    return self._complete(body, chat=True)
                if route in ("/v1/completions", "/completions"):
                    return self._complete(body, chat=False)
                self._json(404, {"error": {"message": f"no route {self.path}"}})
            except BadRequest as e:
                err = {"message": str(e), "type": "invalid_request_error"}
                if e.code:
                    err.update(code=e.code, param=e.param)
                self._json(400, {"error": err})
            except (BrokenPipeError, ConnectionResetError):
                pass
            except Exception as e:  # noqa: BLE001
                try:
                    self._json(500, {"error": {"message": f"{type(e).__name__}: {e}"}})
                except OSError:
                    pass

        def _complete(self, body: dict, chat: bool) -> None:
            prompt = state.chat_prompt(body) if chat else state.completion_prompt(body)
            rid = ("chatcmpl-" if chat else "cmpl-") + uuid.uuid4().hex[:24]
            obj = "chat.completion" if chat else "text_completion"
            created = int(time.time())
            base = {"id": rid, "object": obj + (".chunk" if chat and body.get("stream") else ""), "created": created,
                    "model": state.model_name}
            if body.get("stream"):
                started = [False]

                def on_delta(text: str, ids: list) -> None:
                    if not started[0]:
                        self._sse_start()
                        started[0] = True
                        if chat:
                            self._sse(dict(base, choices=[{"index": 0, "delta": {"role": "assistant"},
                                                           "finish_reason": None}]))
                    if chat:
                        ch = {"index": 0, "delta": {"content": text}, "finish_reason": None}
                    else:
                        ch = {"index": 0, "text": text, "token_ids": ids, "finish_reason": None}
                    self._sse(dict(base, choices=[ch]))

                text, ids, stats, finish = state.generate(prompt, body, on_delta)
                if not started[0]:
                    on_delta("", [])
                last = {"index": 0, "delta": {}, "finish_reason": finish} if chat else \
                    {"index": 0, "text": "", "finish_reason": finish}
                self._sse(dict(base, choices=[last]))
                if (body.get("stream_options") or {}).get("include_usage"):
                    self._sse(dict(base, choices=[], usage=state.usage(stats)))
                self._sse("[DONE]")
                return
            text, ids, stats, finish = state.generate(prompt, body, lambda t, i: None)
            if chat:
                choice = {"index": 0, "message": {"role": "assistant", "content": text}, "finish_reason": finish}
            else:
                choice = {"index": 0, "text": text, "token_ids": ids, "logprobs": None, "finish_reason": finish}
            self._json(200, dict(base, choices=[choice], usage=state.usage(stats)))

    return Handler


def make_server(state: ServerState, host: str = "127.0.0.1", port: int = 8000) -> ThreadingHTTPServer:
    srv = ThreadingHTTPServer((host, port), make_handler(state))
    srv.daemon_threads = True
    return srv


def load_tokenizer(path: Optional[str]):
    """The checkpoint's own tokenizer (local files only), or None."""
    if not path:
        return None
    try:
        from transformers import AutoTokenizer

        return AutoTokenizer.from_pretrained(path, local_files_only=True)
    except Exception:  # noqa: BLE001 - a checkpoint without tokenizer files serves token ids
        return None


def main(argv=None) -> int:
    from .engine import MODES, SHAPES, Engine

    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--model", default="random-tiny", help=f"checkpoint directory or one of {sorted(SHAPES)}")
    ap.add_argument("--mode", choices=MODES, default="self-spec")
    ap.add_argument("--gen-block", type=int, default=None)
    ap.add_argument("--denoise-steps", type=int, default=0)
    ap.add_argument("--host", default="127.0.0.1")
    ap.add_argument("--port", type=int, default=8000)
    ap.add_argument("--context-length", type=int, default=DEFAULTS["context_length"])
    ap.add_argument("--max-tokens", type=int, default=DEFAULTS["max_tokens"])
    ap.add_argument("--temperature", type=float, default=DEFAULTS["temperature"])
    ap.add_argument("--top-k", type=int, default=DEFAULTS["top_k"])
    ap.add_argument("--top-p", type=float, default=DEFAULTS["top_p"])
    ap.add_argument("--prefill-chunk", type=int, default=512)
    ap.add_argument("--no-prompt-cache", action="store_true")
    ap.add_argument("--cache-slots", type=int, default=3,
                    help="conversations whose prompt cache is kept (main loop + side requests)")
    ap.add_argument("--loop-guard", action="store_true",
                    help="stop replies that loop (one block repeated 6+ times, or mostly repeated 16-token "
                         "phrases); reported as finish_reason length")
    args = ap.parse_args(argv)
    from . import decode as _decode

    _decode._Emitter.loop_guard = args.loop_guard
    eng = Engine(args.model, mode=args.mode, gen_block=args.gen_block, denoise_steps=args.denoise_steps,
                 prefill_chunk=args.prefill_chunk, prompt_cache=not args.no_prompt_cache,
                 cache_slots=args.cache_slots)
    state = ServerState(eng, eng.tokenizer, model_name=str(args.model).rstrip("/").split("/")[-1],
                        defaults={"context_length": args.context_length, "max_tokens": args.max_tokens,
                                  "temperature": args.temperature, "top_k": args.top_k, "top_p": args.top_p})
    srv = make_server(state, args.host, args.port)
    print(json.dumps({"listening": f"http://{args.host}:{srv.server_address[1]}", "mode": args.mode}), flush=True)
    try:
        srv.serve_forever()
    except KeyboardInterrupt:
        pass
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
