"""Host-side serving pieces, on the CPU: the OpenAI wire format of the server
(reference server.py:36-227), the streaming benchmark client
(benchmark.py:23-135), incremental detokenization, stop-id selection and
the safetensors weight loader.  The engine is replaced by a scripted fake
that pushes tokens through the same ``Request.sink`` the real scheduler
uses; the GPU engine behind the server is covered by test_gpu_server.py.
"""

from __future__ import annotations

import asyncio
import json
import random
import socket
import threading
import time

import pytest
import torch

from minimal_inference_amd.tokenizer import IncrementalDetokenizer, SyntheticTokenizer, stop_ids

VOCAB = 512
EOS = VOCAB - 1


class FakeScheduler:
    """Emits ``script`` (cut at max_new_tokens) from a thread, then None;
    finish_reason "stop" when a stop id was emitted, as the engine does."""

    max_seq_len = 256

    def __init__(self, script, delay=0.002):
        self.script = list(script)
        self.delay = delay
        self.requests = []
        self.aborted = set()

    def abort_request(self, request_id):
        self.aborted.add(request_id)

    def submit_request(self, req):
        if len(req.input_ids) > self.max_seq_len:
            raise ValueError("prompt too long")
        self.requests.append(req)

        def run():
            out = []
            for t in self.script:
                if req.request_id in self.aborted:
                    req.finish_reason = "abort"
                    req.sink(None)
                    return
                out.append(t)
                req.sink(t)
                time.sleep(self.delay)
                if t == EOS or len(out) >= req.max_new_tokens:
                    break
            req.finish_reason = "stop" if out and out[-1] == EOS else "length"
            req.sink(None)

        threading.Thread(target=run, daemon=True).start()


def _app(script, delay=0.002):
    from minimal_inference_amd.server import create_app

    tok = SyntheticTokenizer(VOCAB)
    sch = FakeScheduler(script, delay)
    return create_app(sch, tok, "fake-model", {EOS}), sch, tok


def _sse(text: str) -> list:
    out = []
    for block in text.split("\n\n"):
        if not block.strip():
            continue
        assert block.startswith("data: ")
        data = block[len("data: "):]
        out.append(data if data == "[DONE]" else json.loads(data))
    return out


SCRIPT = list("héllo wörld ✓".encode()) + [300, 301, EOS, 65, 66]
TEXT = "héllo wörld ✓ w300 w301"


def test_stream_wire_format():
    from fastapi.testclient import TestClient

    app, sch, tok = _app(SCRIPT)
    with TestClient(app) as c:
        r = c.post("/v1/chat/completions", json={"model": "m", "messages": [{"role": "user", "content": "hi"}],
                                                 "max_tokens": 100, "stream": True, "temperature": 0})
        assert r.status_code == 200
        assert r.headers["content-type"].startswith("text/event-stream")
        ev = _sse(r.text)
    assert ev[-1] == "[DONE]"
    chunks = ev[:-1]
    assert all(c["object"] == "chat.completion.chunk" and c["model"] == "m" for c in chunks)
    assert len({c["id"] for c in chunks}) == 1 and chunks[0]["id"].startswith("chatcmpl-")
    assert chunks[0]["choices"][0]["delta"] == {"role": "assistant", "content": None}
    body = chunks[1:-1]
    assert all(c["choices"][0]["finish_reason"] is None and c["choices"][0]["delta"]["content"] for c in body)
    assert "".join(c["choices"][0]["delta"]["content"] for c in body) == TEXT
    # no chunk splits a UTF-8 character: every delta decodes cleanly
    assert all("\ufffd" not in c["choices"][0]["delta"]["content"] for c in body)
    assert chunks[-1]["choices"][0]["finish_reason"] == "stop"
    assert chunks[-1]["choices"][0]["delta"] == {"role": None, "content": None}
    req = sch.requests[0]
    assert req.input_ids == tok.encode("<|user|>\nhi\n<|assistant|>\n")
    assert req.temperature == 0 and req.max_new_tokens == 100 and req.top_p == 1.0


def test_non_stream_response_and_length_finish():
    from fastapi.testclient import TestClient

    app, sch, _ = _app(SCRIPT)
    with TestClient(app) as c:
        r = c.post("/v1/chat/completions", json={"messages": [{"role": "user", "content": "hey"}],
                                                 "max_tokens": 3, "top_p": 0.5})
        assert r.status_code == 200
        j = r.json()
        assert j["object"] == "chat.completion" and j["model"] == "fake-model"
        assert j["choices"][0]["message"] == {"role": "assistant", "content": "hé"}
        assert j["choices"][0]["finish_reason"] == "length"
        n_prompt = len(sch.requests[0].input_ids)
        assert j["usage"] == {"prompt_tokens": n_prompt, "completion_tokens": 3, "total_tokens": n_prompt + 3}
        assert sch.requests[0].top_p == 0.5
        # stop id: excluded from text and from completion_tokens
        r = c.post("/v1/chat/completions", json={"messages": [{"role": "user", "content": "hey"}]})
        j = r.json()
        assert j["choices"][0]["message"]["content"] == TEXT
        assert j["choices"][0]["finish_reason"] == "stop"
        assert j["usage"]["completion_tokens"] == len(SCRIPT) - 3


def test_rejects_bad_requests():
    from fastapi.testclient import TestClient

    app, _, _ = _app(SCRIPT)
    with TestClient(app) as c:
        long = "x" * 400
        r = c.post("/v1/chat/completions", json={"messages": [{"role": "user", "content": long}]})
        assert r.status_code == 400
        r = c.post("/v1/chat/completions", json={"messages": [{"role": "user", "content": "a"}], "max_tokens": 0})
        assert r.status_code == 422
        assert c.get("/v1/models").json()["data"][0]["id"] == "fake-model"
        assert c.get("/health").json() == {"status": "ok"}


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def test_benchmark_client_against_live_server():
    """uvicorn on 127.0.0.1 + the streaming client: chunk counts, TTFT / T2T
    and aggregate figures come out of real SSE over HTTP."""
    import uvicorn

    from minimal_inference_amd.benchmark import run_benchmark

    script = [300 + i for i in range(40)]       # 40 single-piece tokens, no stop id
    app, sch, _ = _app(script)
    port = _free_port()
    server = uvicorn.Server(uvicorn.Config(app, host="127.0.0.1", port=port, log_level="warning"))
    th = threading.Thread(target=server.run, daemon=True)
    th.start()
    try:
        t0 = time.time()
        while not server.started:
            assert time.time() - t0 < 20
            time.sleep(0.05)
        res = asyncio.run(run_benchmark(f"http://127.0.0.1:{port}", max_tokens=25, batch_size=3, runs=2,
                                        verbose=False))
    finally:
        server.should_exit = True
        th.join(10)
    assert len(sch.requests) == 6
    assert all(r.temperature == 0 for r in sch.requests)
    for run in res["per_run"]:
        assert run["tokens"] == 75
        assert all(q["tokens"] == 25 and q["finish_reason"] == "length" for q in run["requests"])
    assert res["ttft_ms"] > 0 and res["t2t_ms"] >= 1.0     # the fake sleeps 2 ms per token
    assert res["aggregate_tok_s"] > 0


# ---------------------------------------------------------------- detokenization
def _check_incremental(tok, ids):
    d = IncrementalDetokenizer(tok)
    parts = [d.push(t) for t in ids]
    parts.append(d.flush())
    assert "".join(parts) == tok.decode(ids, skip_special_tokens=True)
    return parts


def test_incremental_detokenizer_synthetic():
    tok = SyntheticTokenizer(VOCAB)
    rng = random.Random(0)
    text = "ascii, ünïcödé, 漢字, emoji 🌊🐚 and more"
    for _ in range(50):
        ids = tok.encode(text) + [rng.randrange(256, VOCAB - 1) for _ in range(3)]
        rng.shuffle(ids)            # arbitrary byte soup: invalid sequences decode to U+FFFD
        _check_incremental(tok, ids)
    parts = _check_incremental(tok, tok.encode("🌊x"))
    assert parts[:4] == ["", "", "", "🌊"]      # four bytes, one character, emitted once complete


def test_incremental_detokenizer_byte_level_bpe():
    """A byte-level BPE (the tokenizer family of Qwen2 / Mistral v0.3 style
    checkpoints), trained here on a small multilingual text."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    from transformers import PreTrainedTokenizerFast

    corpus = ["The ocean breathes in silver light, waves fold over the shore.",
              "Die Wellen brechen über den Strand, größer und größer.",
              "海の波が岸に寄せては返す。", "Les vagues écument sous la lune. 🌊🐚"] * 20
    bpe = Tokenizer(models.BPE(unk_token=None))
    bpe.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    bpe.decoder = decoders.ByteLevel()
    bpe.train_from_iterator(corpus, trainers.BpeTrainer(vocab_size=400, special_tokens=["<|im_end|>"],
                                                        initial_alphabet=pre_tokenizers.ByteLevel.alphabet()))
    tok = PreTrainedTokenizerFast(tokenizer_object=bpe, eos_token="<|im_end|>")
    for line in corpus[:4]:
        _check_incremental(tok, tok.encode(line))
    rng = random.Random(1)
    for _ in range(30):
        _check_incremental(tok, [rng.randrange(tok.vocab_size) for _ in range(25)])
    assert stop_ids(tok) == {tok.convert_tokens_to_ids("<|im_end|>")}


def test_stop_ids_rules():
    class T:
        eos_token_id = 7
        additional_special_tokens_ids = [9, 11]
        unk_token_id = 0

        def convert_tokens_to_ids(self, s):
            return 0          # unknown -> unk id: not a stop id

    assert stop_ids(T()) == {7, 9, 11}
    assert stop_ids(SyntheticTokenizer(300)) == {299}


# ---------------------------------------------------------------- weights
def test_load_weights_hf_layout(tmp_path):
    """A tiny HF-layout checkpoint (two shards + index) lands in the fused
    q/k/v and gate/up rows; a missing tensor is an error."""
    from safetensors.torch import save_file

    from minimal_inference_amd.model import Model, ModelConfig
    from minimal_inference_amd.weights import load_weights

    raw = {"hidden_size": 32, "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 8,
           "num_hidden_layers": 2, "intermediate_size": 48, "vocab_size": 300, "rms_norm_eps": 1e-6,
           "rope_theta": 10000.0, "tie_word_embeddings": False, "model_type": "qwen2"}
    (tmp_path / "config.json").write_text(json.dumps(raw))
    cfg = ModelConfig.from_pretrained(str(tmp_path))
    assert cfg.attn_bias and not cfg.tie_word_embeddings
    g = torch.Generator().manual_seed(0)
    t = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    sd = {"model.embed_tokens.weight": t(300, 32), "model.norm.weight": t(32), "lm_head.weight": t(300, 32)}
    for i in range(2):
        p = f"model.layers.{i}."
        sd.update({p + "input_layernorm.weight": t(32), p + "post_attention_layernorm.weight": t(32),
                   p + "self_attn.q_proj.weight": t(32, 32), p + "self_attn.q_proj.bias": t(32),
                   p + "self_attn.k_proj.weight": t(16, 32), p + "self_attn.k_proj.bias": t(16),
                   p + "self_attn.v_proj.weight": t(16, 32), p + "self_attn.v_proj.bias": t(16),
                   p + "self_attn.o_proj.weight": t(32, 32), p + "mlp.gate_proj.weight": t(48, 32),
                   p + "mlp.up_proj.weight": t(48, 32), p + "mlp.down_proj.weight": t(32, 48),
                   p + "self_attn.rotary_emb.inv_freq": torch.ones(4)})
    names = sorted(sd)
    shards = {"a.safetensors": names[: len(names) // 2], "b.safetensors": names[len(names) // 2:]}
    for f, ks in shards.items():
        save_file({k: sd[k] for k in ks}, str(tmp_path / f))
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {k: f for f, ks in shards.items() for k in ks}}))
    model = Model(cfg, "cpu", seed=1, max_positions=64)
    load_weights(model, str(tmp_path))
    assert torch.equal(model.embed, sd["model.embed_tokens.weight"])
    assert torch.equal(model.lm_head, sd["lm_head.weight"])
    for i, L in enumerate(model.layers):
        p = f"model.layers.{i}."
        assert torch.equal(L.w_qkv, torch.cat([sd[p + f"self_attn.{n}_proj.weight"] for n in "qkv"]))
        assert torch.equal(L.b_qkv, torch.cat([sd[p + f"self_attn.{n}_proj.bias"] for n in "qkv"]))
        assert torch.equal(L.w_gate_up, torch.cat([sd[p + "mlp.gate_proj.weight"], sd[p + "mlp.up_proj.weight"]]))
        assert torch.equal(L.w_down, sd[p + "mlp.down_proj.weight"])
        assert torch.equal(L.in_norm, sd[p + "input_layernorm.weight"])
    # drop one tensor: the loader refuses
    del sd["model.layers.1.mlp.up_proj.weight"]
    for f in ("a.safetensors", "b.safetensors"):
        (tmp_path / f).unlink()
    (tmp_path / "model.safetensors.index.json").unlink()
    save_file(sd, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="lacks 1 tensors"):
        load_weights(Model(cfg, "cpu", seed=1, max_positions=64), str(tmp_path))


def test_client_disconnect_aborts_request():
    """A streaming client that closes after a few chunks gets its request
    aborted in the engine (the scheduler's abort_request is called)."""
    import httpx
    import uvicorn

    app, sch, _ = _app([300 + i for i in range(200)], delay=0.02)
    port = _free_port()
    server = uvicorn.Server(uvicorn.Config(app, host="127.0.0.1", port=port, log_level="warning"))
    th = threading.Thread(target=server.run, daemon=True)
    th.start()
    try:
        t0 = time.time()
        while not server.started:
            assert time.time() - t0 < 20
            time.sleep(0.05)
        body = {"messages": [{"role": "user", "content": "hi"}], "max_tokens": 200, "stream": True}
        with httpx.stream("POST", f"http://127.0.0.1:{port}/v1/chat/completions", json=body, timeout=30) as r:
            n = 0
            for line in r.iter_lines():
                if line.startswith("data: "):
                    n += 1
                if n >= 4:
                    break
        t0 = time.time()
        while not sch.aborted and time.time() - t0 < 10:
            time.sleep(0.05)
    finally:
        server.should_exit = True
        th.join(10)
    assert sch.aborted == {sch.requests[0].request_id}
