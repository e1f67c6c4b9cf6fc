"""GPU: the OpenAI-compatible server in front of the real engine.

A random-weight Qwen2.5-0.5B-shaped model (4 layers) with the synthetic
tokenizer is served by uvicorn on 127.0.0.1; the streaming benchmark client
sends concurrent greedy requests, with one and with four decode steps per
host round trip.  For every request the streamed text, the number of content
chunks and the finish reason must be exactly what the engine generated for
that request (its ``generated_tokens``), the non-streamed response likewise,
and every request must be retired with its pages returned.  (Token equality
with a separately driven engine is not asserted: a different batch
composition changes the split-K plan and GEMM shapes, so greedy near-ties
may resolve differently.)
"""

from __future__ import annotations

import asyncio
import json
import socket
import threading
import time

import pytest

pytestmark = pytest.mark.gpu

PROMPT = "Write a short poem about the ocean"


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


class _Recorder:
    """Passes requests to the scheduler and keeps them by id."""

    def __init__(self, sch):
        self.sch = sch
        self.by_id = {}

    def submit_request(self, req):
        self.by_id[req.request_id] = req
        self.sch.submit_request(req)

    def abort_request(self, request_id):
        self.sch.abort_request(request_id)

    @property
    def loop_error(self):
        return self.sch.loop_error


@pytest.mark.parametrize("window", [1, 4])
def test_served_streams_match_engine_tokens(dev, window):
    import httpx
    import uvicorn

    from minimal_inference_amd.benchmark import run_benchmark
    from minimal_inference_amd.engine import Scheduler
    from minimal_inference_amd.model import PRESETS, Model
    from minimal_inference_amd.server import create_app
    from minimal_inference_amd.tokenizer import IncrementalDetokenizer, SyntheticTokenizer, stop_ids

    cfg = PRESETS["qwen2.5-0.5b"]
    cfg = type(cfg)(**{**cfg.__dict__, "num_hidden_layers": 4})
    model = Model(cfg, dev, seed=7, max_positions=600)
    tok = SyntheticTokenizer(cfg.vocab_size)
    stops = stop_ids(tok)
    sch = Scheduler(model, max_batch_size=8, max_seq_len=512, eos_token_ids=stops, seed=0, decode_window=window)
    rec = _Recorder(sch)
    sch.start()
    port = _free_port()
    server = uvicorn.Server(uvicorn.Config(create_app(rec, tok, "qwen-test", stops), host="127.0.0.1", port=port,
                                           log_level="warning"))
    th = threading.Thread(target=server.run, daemon=True)
    th.start()
    try:
        t0 = time.time()
        while not server.started:
            assert time.time() - t0 < 30
            time.sleep(0.05)
        url = f"http://127.0.0.1:{port}"
        res = asyncio.run(run_benchmark(url, prompt=PROMPT, max_tokens=20, batch_size=5, runs=2, verbose=False))
        body = {"messages": [{"role": "user", "content": PROMPT}], "max_tokens": 17, "temperature": 0}
        j = httpx.post(url + "/v1/chat/completions", json=body, timeout=60).json()
        health = httpx.get(url + "/health", timeout=10).json()
    finally:
        server.should_exit = True
        th.join(15)
        sch.stop()
    assert sch.loop_error is None and health == {"status": "ok"}

    def expected(req):
        kept = [t for t in req.generated_tokens if t not in stops]
        d = IncrementalDetokenizer(tok)
        chunks = sum(1 for t in kept if d.push(t)) + (1 if d.flush() else 0)
        return tok.decode(kept), chunks, len(kept)

    ids = tok.apply_chat_template([{"role": "user", "content": PROMPT}], tokenize=True)
    for run in res["per_run"]:
        assert len(run["requests"]) == 5
        for q in run["requests"]:
            req = rec.by_id[q["id"]]
            text, chunks, _ = expected(req)
            assert req.input_ids == ids
            assert q["text"] == text and q["tokens"] == chunks
            assert q["finish_reason"] == req.finish_reason
            assert req.finish_reason == "stop" or len(req.generated_tokens) == 20
    req = rec.by_id[j["id"]]
    text, _, n = expected(req)
    assert j["choices"][0]["message"]["content"] == text
    assert j["choices"][0]["finish_reason"] == req.finish_reason
    assert j["usage"] == {"prompt_tokens": len(ids), "completion_tokens": n, "total_tokens": len(ids) + n}
    assert res["t2t_ms"] > 0 and res["ttft_ms"] > 0
    assert not sch.active and not sch.waiting
    assert sch.pt.free_count == sch.kv.max_num_pages - 1              # every request retired


def test_client_disconnect_aborts_in_engine(dev):
    """A streaming client that goes away after a few chunks: the engine
    retires the request with finish_reason "abort" and frees its pages."""
    import httpx
    import uvicorn

    from minimal_inference_amd.engine import Scheduler
    from minimal_inference_amd.model import PRESETS, Model
    from minimal_inference_amd.server import create_app
    from minimal_inference_amd.tokenizer import SyntheticTokenizer, stop_ids

    cfg = PRESETS["qwen2.5-0.5b"]
    model = Model(cfg, dev, seed=7, max_positions=4200)   # 24 layers: ~1 ms per step, 3000 tokens take seconds
    tok = SyntheticTokenizer(cfg.vocab_size)
    stops = stop_ids(tok)
    sch = Scheduler(model, max_batch_size=4, max_seq_len=4096, eos_token_ids=stops, seed=0)
    rec = _Recorder(sch)
    sch.start()
    port = _free_port()
    server = uvicorn.Server(uvicorn.Config(create_app(rec, tok, "qwen-test", stops), host="127.0.0.1", port=port,
                                           log_level="warning"))
    th = threading.Thread(target=server.run, daemon=True)
    th.start()
    try:
        t0 = time.time()
        while not server.started:
            assert time.time() - t0 < 30
            time.sleep(0.05)
        body = {"messages": [{"role": "user", "content": PROMPT}], "max_tokens": 3000, "temperature": 0,
                "stream": True}
        with httpx.stream("POST", f"http://127.0.0.1:{port}/v1/chat/completions", json=body, timeout=60) as r:
            n = 0
            for line in r.iter_lines():
                n += line.startswith("data: ")
                if n >= 5:
                    break
        t0 = time.time()
        while (sch.active or sch.waiting) and time.time() - t0 < 20:
            time.sleep(0.05)
    finally:
        server.should_exit = True
        th.join(15)
        sch.stop()
    (req,) = rec.by_id.values()
    assert req.finish_reason == "abort"
    assert len(req.generated_tokens) < 3000
    assert not sch.active and not sch.waiting
    assert sch.pt.free_count == sch.kv.max_num_pages - 1
