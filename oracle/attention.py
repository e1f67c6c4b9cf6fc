"""Gather-based paged attention in fp32 on the CPU -- oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference's GPU path hands paged decode / prefill attention to an
external library (model.py:235, scheduler.py:402-413, 704-716).  Its own CPU
path states the math it must agree with (model.py:286-295): K/V expanded per
Q head with ``repeat_interleave(group)`` (so Q head h reads KV head
h // group), scaled dot-product attention with the default scale 1/sqrt(d),
causal for prefill.  These functions restate that math over the paged pool:
each request's pages are gathered through kv_indices
(``kv_indices[kv_indptr[b]:kv_indptr[b+1]]``, NHD pool scheduler.py:195-202)
and truncated to kv_len = (npages - 1) * page_size + last_page_len.

Inputs are bf16 (as the kernels see them); all arithmetic is fp32.

Pinning (tests/test_oracle_attention.py): against float64 brute force on
tiny inputs, torch's scaled_dot_product_attention on the gathered tensors,
and closed forms (kv_len 1 -> V[0]; constant logits -> mean of V; one
dominant logit -> that V row; causal row 0 -> V[0]).
"""

from __future__ import annotations

import math

import torch

from .paging import gather_kv


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
            mask: torch.Tensor | None = None) -> torch.Tensor:
    """q [Tq, Hq, D], k/v [Tk, Hkv, D] -> [Tq, Hq, D] in fp32."""
    hq, hkv = q.shape[1], k.shape[1]
    group = hq // hkv
    qf = q.float().transpose(0, 1)  # [Hq, Tq, D]
    kf = k.float().repeat_interleave(group, dim=1).transpose(0, 1)  # model.py:287-288
    vf = v.float().repeat_interleave(group, dim=1).transpose(0, 1)
    logits = torch.matmul(qf, kf.transpose(1, 2)) * scale  # [Hq, Tq, Tk]
    if mask is not None:
        logits = logits.masked_fill(~mask, float("-inf"))
    probs = torch.softmax(logits, dim=-1)
    probs = torch.nan_to_num(probs, nan=0.0)  # rows with no visible key -> 0
    return torch.matmul(probs, vf).transpose(0, 1)


def decode(q: torch.Tensor, pool: torch.Tensor, indptr, indices, last_page_len,
           sm_scale: float | None = None) -> torch.Tensor:
    """Paged decode attention: q [B, Hq, D] bf16, pool [P, 2, ps, Hkv, D] bf16.

    Returns fp32 [B, Hq, D]; rows with kv_len 0 are zero.
    """
    b_count, hq, d = q.shape
    scale = sm_scale if sm_scale else 1.0 / math.sqrt(d)
    out = torch.zeros(b_count, hq, d, dtype=torch.float32)
    for b in range(b_count):
        k, v = gather_kv(pool, indptr, indices, last_page_len, b)
        if k.shape[0] == 0:
            continue
        out[b] = _attend(q[b:b + 1], k, v, scale)[0]
    return out


def prefill(q: torch.Tensor, pool: torch.Tensor, qo_indptr, kv_indptr, indices, last_page_len,
            causal: bool = True, sm_scale: float | None = None) -> torch.Tensor:
    """Ragged paged prefill: q [total_q, Hq, D] -> fp32 [total_q, Hq, D].

    Query row i of request b sees KV token j when j <= i + (kv_len - qo_len)
    (bottom-right aligned causal mask; the reference always has kv == qo).
    """
    d = q.shape[2]
    scale = sm_scale if sm_scale else 1.0 / math.sqrt(d)
    out = torch.zeros(q.shape, dtype=torch.float32)
    nb = len(qo_indptr) - 1
    for b in range(nb):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        if q1 == q0:
            continue
        k, v = gather_kv(pool, kv_indptr, indices, last_page_len, b)
        kv_len, qo_len = k.shape[0], q1 - q0
        if kv_len == 0:
            continue
        mask = None
        if causal:
            i = torch.arange(qo_len).unsqueeze(1)
            j = torch.arange(kv_len).unsqueeze(0)
            mask = (j <= i + (kv_len - qo_len)).unsqueeze(0)  # [1, Tq, Tk]
        out[q0:q1] = _attend(q[q0:q1], k, v, scale, mask)
    return out
