"""OpenAI-compatible ``/v1/chat/completions`` server over the engine.

Same wire format as the reference's server (server.py:36-89 schema,
127-227 endpoint): JSON responses, or with ``"stream": true`` server-sent
events -- a first chunk carrying ``{"role": "assistant"}``, one chunk per
non-empty text delta, a last chunk with an empty delta and the
``finish_reason`` ("stop" after a stop id, which is not sent as text,
otherwise "length"), then ``data: [DONE]``.  Additions: an optional
``top_p`` field, ``GET /v1/models`` and ``GET /health``; prompts that can
never fit (longer than ``max_seq_len`` or the pool) are answered with 400;
a request whose client goes away is aborted in the engine (the reference
keeps generating for it).

The engine (``engine.Scheduler``) runs its step loop in a daemon thread and
pushes each token into the request's asyncio queue with
``loop.call_soon_threadsafe``, ``None`` when the request is retired.

Run:  python minimal-inference_amd/server.py --config server_config.yaml
Config keys (the reference's config.yaml plus a few): ``model_path`` (HF
checkpoint directory) or ``model_preset`` (random weights of a named
architecture, with the synthetic tokenizer), ``device``, ``dtype``
(bfloat16), ``seed``, ``server.host`` / ``server.port``,
``scheduler.max_seq_len`` / ``max_batch_size`` / ``page_size`` /
``decode_window`` / ``pipeline`` / ``use_graphs`` (``use_flashinfer`` is
accepted and ignored: the HIP path is the only one).
"""

from __future__ import annotations

if __name__ == "__main__" and not __package__:
    # launched as a script: import the package from its directory, then run
    import importlib.util as _ilu
    import sys as _sys
    from pathlib import Path as _Path

    _dir = _Path(__file__).resolve().parent
    if "minimal_inference_amd" not in _sys.modules:
        _spec = _ilu.spec_from_file_location("minimal_inference_amd", _dir / "__init__.py",
                                             submodule_search_locations=[str(_dir)])
        _pkg = _ilu.module_from_spec(_spec)
        _sys.modules["minimal_inference_amd"] = _pkg
        _spec.loader.exec_module(_pkg)
    from minimal_inference_amd.server import main as _main

    _sys.exit(_main())

import argparse
import asyncio
import logging
import os
import time
import uuid

from fastapi import FastAPI, HTTPException
from fastapi.middleware.cors import CORSMiddleware
from fastapi.responses import StreamingResponse
from pydantic import BaseModel, Field

from .engine import Request
from .tokenizer import IncrementalDetokenizer

log = logging.getLogger("minimal_inference_amd.server")


# ---------------------------------------------------------------- OpenAI schema
class ChatMessage(BaseModel):
    role: str
    content: str


class ChatCompletionRequest(BaseModel):
    model: str = ""
    messages: list[ChatMessage]
    temperature: float = 0.7
    max_tokens: int = Field(512, ge=1)
    stream: bool = False
    top_p: float = Field(1.0, gt=0.0, le=1.0)


class Choice(BaseModel):
    index: int = 0
    message: ChatMessage
    finish_reason: str


class Usage(BaseModel):
    prompt_tokens: int
    completion_tokens: int
    total_tokens: int


class ChatCompletionResponse(BaseModel):
    id: str
    object: str = "chat.completion"
    created: int
    model: str
    choices: list[Choice]
    usage: Usage


class DeltaMessage(BaseModel):
    role: str | None = None
    content: str | None = None


class StreamChoice(BaseModel):
    index: int = 0
    delta: DeltaMessage
    finish_reason: str | None = None


class ChatCompletionChunk(BaseModel):
    id: str
    object: str = "chat.completion.chunk"
    created: int
    model: str
    choices: list[StreamChoice]


# ---------------------------------------------------------------- app
def create_app(scheduler, tokenizer, model_name: str, stop_ids: set[int]) -> FastAPI:
    """``scheduler`` needs ``submit_request(Request)`` and a running loop
    (``engine.Scheduler`` after ``start()``); tokens reach each request
    through its ``sink``."""
    app = FastAPI(title="minimal-inference (MI355X)")
    app.add_middleware(CORSMiddleware, allow_origins=["*"], allow_methods=["*"], allow_headers=["*"])
    stops = set(stop_ids)

    def prompt_ids(messages: list[ChatMessage]) -> list[int]:
        text = tokenizer.apply_chat_template([m.model_dump() for m in messages], tokenize=False,
                                             add_generation_prompt=True)
        return tokenizer.encode(text)

    @app.get("/health")
    async def health():
        err = getattr(scheduler, "loop_error", None)
        if err is not None:
            raise HTTPException(503, f"engine stopped: {err!r}")
        return {"status": "ok"}

    @app.get("/v1/models")
    async def models():
        return {"object": "list", "data": [{"id": model_name, "object": "model", "owned_by": "local"}]}

    @app.post("/v1/chat/completions")
    async def chat_completions(body: ChatCompletionRequest):
        loop = asyncio.get_running_loop()
        queue: asyncio.Queue = asyncio.Queue()
        req = Request(request_id=f"chatcmpl-{uuid.uuid4().hex[:12]}", input_ids=prompt_ids(body.messages),
                      max_new_tokens=body.max_tokens, temperature=body.temperature, top_p=body.top_p,
                      sink=lambda t: loop.call_soon_threadsafe(queue.put_nowait, t))
        try:
            scheduler.submit_request(req)
        except ValueError as e:
            raise HTTPException(400, str(e))
        except RuntimeError as e:
            raise HTTPException(503, str(e))
        name = body.model or model_name
        if body.stream:
            return StreamingResponse(_stream(req, queue, name), media_type="text/event-stream")
        return await _complete(req, queue, name)

    def abort(req: Request) -> None:
        fn = getattr(scheduler, "abort_request", None)
        if fn is not None:
            fn(req.request_id)

    async def _complete(req: Request, queue: asyncio.Queue, name: str) -> ChatCompletionResponse:
        ids: list[int] = []
        finish = "length"
        try:
            while True:
                t = await queue.get()
                if t is None:
                    finish = req.finish_reason or finish
                    break
                if t in stops:
                    finish = "stop"
                    continue
                ids.append(t)
        except asyncio.CancelledError:  # the client went away
            abort(req)
            raise
        if finish == "error":
            raise HTTPException(500, "engine error")
        return ChatCompletionResponse(
            id=req.request_id, created=int(time.time()), model=name,
            choices=[Choice(message=ChatMessage(role="assistant",
                                                content=tokenizer.decode(ids, skip_special_tokens=True)),
                            finish_reason=finish)],
            usage=Usage(prompt_tokens=len(req.input_ids), completion_tokens=len(ids),
                        total_tokens=len(req.input_ids) + len(ids)))

    async def _stream(req: Request, queue: asyncio.Queue, name: str):
        created = int(time.time())

        def chunk(delta: DeltaMessage, finish: str | None = None) -> str:
            c = ChatCompletionChunk(id=req.request_id, created=created, model=name,
                                    choices=[StreamChoice(delta=delta, finish_reason=finish)])
            return f"data: {c.model_dump_json()}\n\n"

        done = False
        try:
            yield chunk(DeltaMessage(role="assistant"))
            detok = IncrementalDetokenizer(tokenizer)
            finish = "length"
            while True:
                t = await queue.get()
                if t is None:
                    done = True
                    finish = req.finish_reason or finish
                    break
                if t in stops:
                    finish = "stop"
                    continue
                text = detok.push(t)
                if text:
                    yield chunk(DeltaMessage(content=text))
        finally:
            if not done:  # closed early: the client disconnected
                abort(req)
        tail = detok.flush()
        if tail:
            yield chunk(DeltaMessage(content=tail))
        yield chunk(DeltaMessage(), finish=finish)
        yield "data: [DONE]\n\n"

    return app


# ---------------------------------------------------------------- engine from a config
def init_engine(config: dict):
    """(scheduler started, tokenizer, model name, stop ids) from a config
    dict shaped like the reference's config.yaml (server.py:235-285)."""
    import torch

    from .engine import Scheduler
    from .model import PRESETS, Model, ModelConfig
    from .tokenizer import SyntheticTokenizer, load_tokenizer, stop_ids

    if str(config.get("dtype", "bfloat16")) not in ("bfloat16", "bf16"):
        raise ValueError("the HIP path computes in bfloat16; set dtype: bfloat16")
    dev = torch.device(config.get("device", "cuda"))
    if dev.type != "cuda":
        raise ValueError("the server runs on a GPU (device: cuda or cuda:N)")
    if dev.index is None:
        dev = torch.device("cuda", 0)
    sc = config.get("scheduler", {})
    max_seq = int(sc.get("max_seq_len", 4096))
    model_path = config.get("model_path")
    seed = int(config.get("seed", 0))
    if model_path:
        from .weights import load_weights

        cfg = ModelConfig.from_pretrained(model_path)
        model = Model(cfg, dev, seed=seed, max_positions=max_seq + 16)
        load_weights(model, model_path)
        tok = load_tokenizer(model_path)
        name = os.path.basename(model_path.rstrip("/")).lower()
    else:
        preset = config.get("model_preset", "qwen2.5-0.5b")
        cfg = PRESETS[preset]
        model = Model(cfg, dev, seed=seed, max_positions=max_seq + 16)
        tok = SyntheticTokenizer(cfg.vocab_size)
        name = f"{preset}-random"
    stops = stop_ids(tok)
    sch = Scheduler(model, max_batch_size=int(sc.get("max_batch_size", 40)), max_seq_len=max_seq,
                    page_size=int(sc.get("page_size", 16)), eos_token_ids=stops or None,
                    use_graphs=bool(sc.get("use_graphs", True)), seed=seed,
                    decode_window=int(sc.get("decode_window", 1)), pipeline=bool(sc.get("pipeline", False)))
    sch.start()
    return sch, tok, name, stops


def main(argv=None) -> int:
    import uvicorn
    import yaml

    logging.basicConfig(level=logging.INFO, format="%(name)s - %(message)s")
    ap = argparse.ArgumentParser(description="OpenAI-compatible server on the MI355X paged-attention engine")
    ap.add_argument("--config", default=os.path.join(os.path.dirname(__file__), "server_config.yaml"))
    ap.add_argument("--host", default=None)
    ap.add_argument("--port", type=int, default=None)
    args = ap.parse_args(argv)
    with open(args.config) as f:
        config = yaml.safe_load(f)
    sch, tok, name, stops = init_engine(config)
    srv = config.get("server", {})
    log.info("engine ready: model=%s, max_batch_size=%d, page_size=%d, decode_window=%d", name,
             sch.max_batch_size, sch.page_size, sch.decode_window)
    uvicorn.run(create_app(sch, tok, name, stops), host=args.host or srv.get("host", "127.0.0.1"),
                port=args.port or int(srv.get("port", 8000)), log_level="warning")
    sch.stop()
    return 0
