"""Dense Qwen2 / Mistral transformer driving the paged-attention path.

Restates model.py of the reference (ModelConfig 37-71, RoPE 79-107, RMSNorm
115-122, Attention 126-252, MLP 301-311, DecoderLayer 314-344, Model
352-435).  Dense GEMMs, RMSNorm and RoPE stay on PyTorch-ROCm (hipBLASLt);
the attention layer calls the HIP library through the reference's drop-in
surface: ``append_paged_kv_cache`` then ``wrapper.run`` (model.py:207-235),
without the reference's Q-head padding (model.py:134-137, 226-243): any
integer GQA group runs natively.

Layout choices (dense path only; numerics match the separate-projection
form): q/k/v projections are one fused GEMM and gate/up one fused GEMM, and
prefill computes logits only for each request's last position.  By default
RoPE on q and k and the K/V append run as one HIP launch
(``rope_append_paged_kv_cache``), bit-identical to the reference's bf16
RoPE ops followed by the append, and in decode steps the attention launch
does both itself (``run_rope_append``; ``fused_decode=False`` keeps the
separate launch), bit-identical again; ``fused_rope=False`` keeps the
separate ops.
By default the residual adds and the RMSNorms that follow them run as one
HIP kernel each, and SiLU(gate) * up as one (``dense.add_rms_norm`` /
``dense.silu_mul``, fp32 math, one bf16 rounding per output);
``fused_dense=False`` keeps torch's ``F.rms_norm``, adds and
``F.silu(g) * u``.  RoPE tables are held in the model dtype, as the reference's are after ``.to(dtype)``
(server.py:251).  Weights are random-initialised on the device (N(0, 0.02),
norms 1) -- the benchmark configurations use random weights.
"""

from __future__ import annotations

import dataclasses
import json
import math
import os

import torch
import torch.nn.functional as F

from .dense import add_rms_norm, silu_mul
from .page import append_paged_kv_cache, rope_append_paged_kv_cache


@dataclasses.dataclass
class ModelConfig:
    hidden_size: int = 896
    num_attention_heads: int = 14
    num_key_value_heads: int = 2
    head_dim: int = 64
    num_hidden_layers: int = 24
    intermediate_size: int = 4864
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = True
    attn_bias: bool = True

    @classmethod
    def from_pretrained(cls, model_path: str) -> "ModelConfig":
        """Same field mapping as the reference (model.py:52-71)."""
        with open(os.path.join(model_path, "config.json")) as f:
            raw = json.load(f)
        return cls(
            hidden_size=raw["hidden_size"],
            num_attention_heads=raw["num_attention_heads"],
            num_key_value_heads=raw["num_key_value_heads"],
            head_dim=raw.get("head_dim", raw["hidden_size"] // raw["num_attention_heads"]),
            num_hidden_layers=raw["num_hidden_layers"],
            intermediate_size=raw["intermediate_size"],
            vocab_size=raw["vocab_size"],
            rms_norm_eps=raw.get("rms_norm_eps", 1e-6),
            rope_theta=raw.get("rope_theta", 1_000_000.0),
            max_position_embeddings=raw.get("max_position_embeddings", 32768),
            tie_word_embeddings=raw.get("tie_word_embeddings", True),
            attn_bias=raw.get("attention_bias", raw.get("model_type", "") != "mistral"),
        )

    @property
    def group(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads


# Architectures of the benchmark workloads (random-initialised weights).
PRESETS: dict[str, ModelConfig] = {
    "qwen2.5-0.5b": ModelConfig(),
    "mistral-7b": ModelConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                              num_hidden_layers=32, intermediate_size=14336, vocab_size=32768,
                              rms_norm_eps=1e-5, rope_theta=1_000_000.0, tie_word_embeddings=False,
                              attn_bias=False),
    "qwen2.5-7b": ModelConfig(hidden_size=3584, num_attention_heads=28, num_key_value_heads=4, head_dim=128,
                              num_hidden_layers=28, intermediate_size=18944, vocab_size=152064,
                              tie_word_embeddings=False, attn_bias=True),
    "qwen2.5-72b": ModelConfig(hidden_size=8192, num_attention_heads=64, num_key_value_heads=8, head_dim=128,
                               num_hidden_layers=80, intermediate_size=29568, vocab_size=152064,
                               tie_word_embeddings=False, attn_bias=True),
}


def precompute_rope(head_dim: int, max_len: int, theta: float, device, dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin tables [max_len, head_dim] (model.py:79-89), cast to ``dtype``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    t = torch.arange(max_len, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE (model.py:92-107); x [T, H, D], cos/sin [T, D]."""
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos.unsqueeze(1) + rotated * sin.unsqueeze(1)


class Layer:
    def __init__(self, cfg: ModelConfig, device, dtype, gen: torch.Generator):
        h, d = cfg.hidden_size, cfg.head_dim
        nq, nkv = cfg.num_attention_heads, cfg.num_key_value_heads
        std = 0.02

        def w(*shape):
            return (torch.randn(*shape, device=device, dtype=torch.float32, generator=gen) * std).to(dtype)

        self.in_norm = torch.ones(h, device=device, dtype=dtype)
        self.post_norm = torch.ones(h, device=device, dtype=dtype)
        self.w_qkv = w((nq + 2 * nkv) * d, h)
        self.b_qkv = w((nq + 2 * nkv) * d) if cfg.attn_bias else None
        self.w_o = w(h, nq * d)
        self.w_gate_up = w(2 * cfg.intermediate_size, h)
        self.w_down = w(h, cfg.intermediate_size)


@dataclasses.dataclass
class AttentionBackend:
    """What the attention layers need for one forward (scheduler.py:229-259).

    ``wrapper`` is a planned decode or prefill wrapper; ``kv_indices`` /
    ``kv_indptr`` / ``kv_last_page_len`` are the CSR page table;
    ``batch_indices`` / ``positions`` place each new token's K/V.
    ``append_indptr`` is carried for interface parity (unused, as in the
    reference).
    """

    paged_kv_cache: object
    wrapper: object
    mode: str
    kv_page_indptr: torch.Tensor
    kv_page_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    append_indptr: torch.Tensor | None
    batch_indices: torch.Tensor
    positions: torch.Tensor
    _layer_idx: int = 0

    def next_layer(self) -> int:
        idx = self._layer_idx
        self._layer_idx += 1
        return idx


class Model:
    def __init__(self, cfg: ModelConfig, device, dtype=torch.bfloat16, seed: int = 0, max_positions: int | None = None,
                 fused_rope: bool = True, fused_dense: bool = True, fused_decode: bool = True):
        self.cfg = cfg
        self.fused_rope = fused_rope
        self.fused_decode = fused_decode
        self.fused_dense = fused_dense
        self.device = torch.device(device)
        self.dtype = dtype
        gen = torch.Generator(device=self.device).manual_seed(seed)
        self.embed = (torch.randn(cfg.vocab_size, cfg.hidden_size, device=self.device, generator=gen) * 0.02).to(dtype)
        self.layers = [Layer(cfg, self.device, dtype, gen) for _ in range(cfg.num_hidden_layers)]
        self.norm = torch.ones(cfg.hidden_size, device=self.device, dtype=dtype)
        self.lm_head = self.embed if cfg.tie_word_embeddings else \
            (torch.randn(cfg.vocab_size, cfg.hidden_size, device=self.device, generator=gen) * 0.02).to(dtype)
        n = max_positions or cfg.max_position_embeddings
        self.cos, self.sin = precompute_rope(cfg.head_dim, n, cfg.rope_theta, self.device, dtype)

    def weight_bytes(self) -> int:
        t = self.embed.numel() + self.norm.numel()
        if self.lm_head is not self.embed:
            t += self.lm_head.numel()
        for L in self.layers:
            for x in (L.in_norm, L.post_norm, L.w_qkv, L.b_qkv, L.w_o, L.w_gate_up, L.w_down):
                if x is not None:
                    t += x.numel()
        return t * self.embed.element_size()

    # ------------------------------------------------------------------ forward
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, backend: AttentionBackend,
                last_rows: torch.Tensor | None = None) -> torch.Tensor:
        """input_ids / positions: [T] (one row per new token).

        Decode: T = batch, returns logits [T, V].  Prefill: T = sum of prompt
        lengths, returns logits [len(last_rows), V] for the rows given.
        """
        cfg = self.cfg
        nq, nkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        x = F.embedding(input_ids, self.embed)
        fused = self.fused_rope
        if fused:
            rope_pos = positions if positions.dtype == torch.int32 else positions.to(torch.int32)
        else:
            cos = self.cos.index_select(0, positions)
            sin = self.sin.index_select(0, positions)
        t = input_ids.shape[0]
        backend._layer_idx = 0
        eps = cfg.rms_norm_eps
        dense = self.fused_dense
        if dense:
            h = add_rms_norm(x, None, self.layers[0].in_norm, eps, write_x=False)
        for li, L in enumerate(self.layers):
            layer_idx = backend.next_layer()
            if not dense:
                h = F.rms_norm(x, (cfg.hidden_size,), L.in_norm, eps)
            qkv = F.linear(h, L.w_qkv, L.b_qkv)
            kv_data = backend.paged_kv_cache.kv_data[layer_idx]
            if fused and backend.mode == "decode" and self.fused_decode:
                # RoPE, append and attention in one launch (one new token per
                # request, at its last position)
                o = backend.wrapper.run_rope_append(qkv, self.cos, self.sin, kv_data)
            elif fused:
                # q rotated in place in qkv's q columns; k rotated and v appended
                q = rope_append_paged_kv_cache(qkv, nq, nkv, rope_pos, self.cos, self.sin, backend.batch_indices,
                                               backend.positions, kv_data, backend.kv_page_indices,
                                               backend.kv_page_indptr, backend.kv_last_page_len)
            else:
                q = apply_rope(qkv[:, : nq * d].view(t, nq, d), cos, sin)
                k = apply_rope(qkv[:, nq * d: (nq + nkv) * d].view(t, nkv, d), cos, sin)
                v = qkv[:, (nq + nkv) * d:].view(t, nkv, d)
                append_paged_kv_cache(k, v, backend.batch_indices, backend.positions, kv_data,
                                      backend.kv_page_indices, backend.kv_page_indptr, backend.kv_last_page_len)
            if not (fused and backend.mode == "decode" and self.fused_decode):
                o = backend.wrapper.run(q, kv_data)
            if not dense:
                x = x + F.linear(o.view(t, nq * d), L.w_o)
                h = F.rms_norm(x, (cfg.hidden_size,), L.post_norm, eps)
                gu = F.linear(h, L.w_gate_up)
                g, u = gu.chunk(2, dim=-1)
                x = x + F.linear(F.silu(g) * u, L.w_down)
                continue
            # x += o W_o; h = rms(x); x += down(silu(g) * u); h = next layer's rms(x)
            h = add_rms_norm(x, F.linear(o.view(t, nq * d), L.w_o), L.post_norm, eps)
            down = F.linear(silu_mul(F.linear(h, L.w_gate_up)), L.w_down)
            if li + 1 < len(self.layers):
                h = add_rms_norm(x, down, self.layers[li + 1].in_norm, eps)
            elif last_rows is None:
                h = add_rms_norm(x, down, self.norm, eps)
            else:
                add_rms_norm(x, down, None, eps, norm=False)
                h = add_rms_norm(x.index_select(0, last_rows), None, self.norm, eps, write_x=False)
        if not dense:
            if last_rows is not None:
                x = x.index_select(0, last_rows)
            h = F.rms_norm(x, (cfg.hidden_size,), self.norm, eps)
        return F.linear(h, self.lm_head)


def kv_pool_bytes_per_page(cfg: ModelConfig, page_size: int = 16) -> int:
    return 2 * page_size * cfg.num_key_value_heads * cfg.head_dim * 2 * cfg.num_hidden_layers


def default_pages(cfg: ModelConfig, max_batch: int, max_seq_len: int, page_size: int = 16) -> int:
    return max_batch * math.ceil(max_seq_len / page_size)
