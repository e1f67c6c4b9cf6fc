"""Transformer forward on the CPU over the paged KV pool -- oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates the reference's model forward on the CPU for the CPU baseline of the
end-to-end decode (bench.py) and as a checker:

* ``rms_norm`` -- RMSNorm (model.py:115-122): x * rsqrt(mean(x^2) + eps) * w;
* ``rope`` -- rotate-half RoPE (model.py:92-107) with cos / sin rows taken at
  the token positions (model.py:399-400), here in fp32;
* ``decode_step`` -- one decode step of the whole model (Model.forward,
  model.py:375-426; DecoderLayer 314-344; MLP 301-311): per layer RMSNorm,
  q/k/v projection with bias where the model has one, RoPE on q and k, the
  new token's K / V appended to its slot of the layer's paged pool
  (model.py:207-216), gather-based paged attention over the request's pages
  (``oracle.attention.decode``, the math of model.py:254-298), o_proj,
  residual, RMSNorm, SiLU-gated MLP, residual; final RMSNorm and the LM head;
* ``prefill_step`` -- the batched ragged prefill of whole prompts: every
  prompt token's K / V written to its slot, paged causal attention
  (``oracle.attention.prefill``), logits of each prompt's last token;
* ``dense_forward`` -- the same model over a whole sequence with causal
  attention on dense K / V (no pages), used to pin ``decode_step`` and
  ``prefill_step``.

Weights are plain CPU tensors (any float dtype; the arithmetic is fp32):
``embed [V, H]``, ``lm_head [V, H]``, ``norm [H]`` and per layer ``in_norm``,
``post_norm [H]``, ``w_qkv [(Hq + 2 Hkv) D, H]``, ``b_qkv`` (or None),
``w_o [H, Hq D]``, ``w_gate_up [2 I, H]`` (gate rows first), ``w_down [H, I]``.

Pinning (tests/test_oracle_model.py): ``decode_step`` run token by token after
a prompt equals ``dense_forward`` of the same sequence at every new position
(two formulations: paged gather vs dense causal SDPA, incremental vs whole
sequence); ``prefill_step`` of a ragged batch equals ``dense_forward`` of each
prompt at its last position, and decode steps after it continue the dense
forward; ``rms_norm`` against its float64 closed form and a constant-row
case; ``rope`` by position 0 being the identity and the plane-rotation closed
form.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from .attention import decode as paged_decode
from .attention import prefill as paged_prefill


@dataclass
class Shape:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1_000_000.0


@dataclass
class Weights:
    embed: torch.Tensor
    lm_head: torch.Tensor
    norm: torch.Tensor
    layers: list = field(default_factory=list)  # dicts: in_norm, post_norm, w_qkv, b_qkv, w_o, w_gate_up, w_down


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def rope(x: torch.Tensor, positions: torch.Tensor, head_dim: int, theta: float) -> torch.Tensor:
    """x [T, H, D] fp32, positions [T] -> rotated x (fp32)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    freqs = torch.outer(positions.double(), inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos().float().unsqueeze(1), emb.sin().float().unsqueeze(1)
    half = head_dim // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rotated * sin


def _mlp(h: torch.Tensor, L: dict) -> torch.Tensor:
    gu = h @ L["w_gate_up"].float().T
    g, u = gu.chunk(2, dim=-1)
    return (F.silu(g) * u) @ L["w_down"].float().T


def _qkv(h: torch.Tensor, L: dict, s: Shape):
    qkv = h @ L["w_qkv"].float().T
    if L.get("b_qkv") is not None:
        qkv = qkv + L["b_qkv"].float()
    t, d = h.shape[0], s.head_dim
    q = qkv[:, : s.heads * d].view(t, s.heads, d)
    k = qkv[:, s.heads * d: (s.heads + s.kv_heads) * d].view(t, s.kv_heads, d)
    v = qkv[:, (s.heads + s.kv_heads) * d:].view(t, s.kv_heads, d)
    return q, k, v


def decode_step(w: Weights, s: Shape, ids: torch.Tensor, positions: torch.Tensor, pools: list,
                indptr: list, indices: list, last_page_len: list, page_size: int = 16) -> torch.Tensor:
    """One decode token per request: ids / positions [B]; ``pools[l]`` is
    layer l's pool ``[P, 2, page_size, Hkv, D]`` (written in place: the new
    token's K / V go to its slot); the CSR describes each request including
    the new token.  Returns fp32 logits [B, V]."""
    b = ids.shape[0]
    x = w.embed[ids].float()
    pos = positions.long()
    slots = []
    for r in range(b):
        p = int(pos[r])
        slots.append((indices[indptr[r] + p // page_size], p % page_size))
    for li, L in enumerate(w.layers):
        h = rms_norm(x, L["in_norm"], s.eps)
        q, k, v = _qkv(h, L, s)
        q = rope(q, pos, s.head_dim, s.theta)
        k = rope(k, pos, s.head_dim, s.theta)
        pool = pools[li]
        for r, (pg, off) in enumerate(slots):
            pool[pg, 0, off] = k[r].to(pool.dtype)
            pool[pg, 1, off] = v[r].to(pool.dtype)
        o = paged_decode(q.to(pool.dtype), pool, indptr, indices, last_page_len)
        x = x + o.reshape(b, -1) @ L["w_o"].float().T
        x = x + _mlp(rms_norm(x, L["post_norm"], s.eps), L)
    return rms_norm(x, w.norm, s.eps) @ w.lm_head.float().T


def prefill_step(w: Weights, s: Shape, ids: torch.Tensor, qo_indptr: list, pools: list, indptr: list,
                 indices: list, last_page_len: list, page_size: int = 16) -> torch.Tensor:
    """Ragged causal prefill of whole prompts (the batched form of
    scheduler.py:684-752): ``ids`` [T] holds the prompts back to back
    (``qo_indptr``), prompt b at positions 0..L_b-1; the CSR describes each
    request's pages (kv_len = L_b).  Every prompt token's K / V is written to
    its slot of ``pools[l]``; attention is the oracle's paged causal prefill.
    Returns fp32 logits of each prompt's last token [B, V]."""
    nb = len(qo_indptr) - 1
    lens = [qo_indptr[b + 1] - qo_indptr[b] for b in range(nb)]
    pos = torch.cat([torch.arange(n) for n in lens])
    pg = torch.tensor([indices[indptr[b] + p // page_size] for b in range(nb) for p in range(lens[b])])
    off = pos % page_size
    x = w.embed[ids].float()
    for li, L in enumerate(w.layers):
        h = rms_norm(x, L["in_norm"], s.eps)
        q, k, v = _qkv(h, L, s)
        q = rope(q, pos, s.head_dim, s.theta)
        k = rope(k, pos, s.head_dim, s.theta)
        pool = pools[li]
        pool[pg, 0, off] = k.to(pool.dtype)
        pool[pg, 1, off] = v.to(pool.dtype)
        o = paged_prefill(q.to(pool.dtype), pool, qo_indptr, indptr, indices, last_page_len, causal=True)
        x = x + o.reshape(x.shape[0], -1) @ L["w_o"].float().T
        x = x + _mlp(rms_norm(x, L["post_norm"], s.eps), L)
    last = torch.tensor([qo_indptr[b + 1] - 1 for b in range(nb)])
    return rms_norm(x[last], w.norm, s.eps) @ w.lm_head.float().T


def dense_forward(w: Weights, s: Shape, ids: torch.Tensor) -> torch.Tensor:
    """Causal forward over one whole sequence ids [T] (positions 0..T-1),
    K / V kept dense; returns fp32 logits [T, V]."""
    t = ids.shape[0]
    pos = torch.arange(t)
    x = w.embed[ids].float()
    g = s.heads // s.kv_heads
    for L in w.layers:
        h = rms_norm(x, L["in_norm"], s.eps)
        q, k, v = _qkv(h, L, s)
        q = rope(q, pos, s.head_dim, s.theta).transpose(0, 1)
        k = rope(k, pos, s.head_dim, s.theta).repeat_interleave(g, dim=1).transpose(0, 1)
        v = v.repeat_interleave(g, dim=1).transpose(0, 1)
        logits = (q @ k.transpose(1, 2)) / math.sqrt(s.head_dim)
        mask = torch.ones(t, t, dtype=torch.bool).tril()
        o = torch.softmax(logits.masked_fill(~mask, float("-inf")), dim=-1) @ v
        x = x + o.transpose(0, 1).reshape(t, -1) @ L["w_o"].float().T
        x = x + _mlp(rms_norm(x, L["post_norm"], s.eps), L)
    return rms_norm(x, w.norm, s.eps) @ w.lm_head.float().T


def random_weights(s: Shape, layers: int, seed: int = 0, bias: bool = True) -> Weights:
    """N(0, 0.02) weights, norms 1 (the benchmark workloads' initialisation)."""
    g = torch.Generator().manual_seed(seed)
    d = s.head_dim

    def rnd(*shape):
        return torch.randn(*shape, generator=g) * 0.02

    lay = []
    for _ in range(layers):
        lay.append({"in_norm": torch.ones(s.hidden), "post_norm": torch.ones(s.hidden),
                    "w_qkv": rnd((s.heads + 2 * s.kv_heads) * d, s.hidden),
                    "b_qkv": rnd((s.heads + 2 * s.kv_heads) * d) if bias else None,
                    "w_o": rnd(s.hidden, s.heads * d), "w_gate_up": rnd(2 * s.intermediate, s.hidden),
                    "w_down": rnd(s.hidden, s.intermediate)})
    return Weights(embed=rnd(s.vocab, s.hidden), lm_head=rnd(s.vocab, s.hidden), norm=torch.ones(s.hidden),
                   layers=lay)
