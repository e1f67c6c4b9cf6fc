"""Seeded synthetic inputs shared by the CPU and GPU tests."""

from __future__ import annotations

import math

import torch


def make_paged_batch(lens, hq, hkv, d, num_pages=None, page_size=16, seed=0, scale=1.0):
    """Pool + CSR for requests of the given lengths, pages from a permutation.

    Returns dict with pool [P,2,ps,hkv,d] bf16, q [B,hq,d] bf16, indptr (list),
    indices (int32 tensor), last (list).
    """
    g = torch.Generator().manual_seed(seed)
    npages = [math.ceil(n / page_size) for n in lens]
    total = sum(npages)
    num_pages = num_pages or max(total + 1, 8)
    pool = (torch.randn(num_pages, 2, page_size, hkv, d, generator=g) * scale).to(torch.bfloat16)
    perm = torch.randperm(num_pages, generator=g)
    indptr = [0]
    for n in npages:
        indptr.append(indptr[-1] + n)
    indices = perm[:total].to(torch.int32)
    last = [(n - (p - 1) * page_size) if p > 0 else 0 for n, p in zip(lens, npages)]
    q = (torch.randn(len(lens), hq, d, generator=g) * scale).to(torch.bfloat16)
    return {"pool": pool, "q": q, "indptr": indptr, "indices": indices, "last": last}


def to_dev(batch, dev):
    return (
        batch["pool"].to(dev),
        batch["q"].to(dev),
        torch.tensor(batch["indptr"], dtype=torch.int32, device=dev),
        batch["indices"].to(dev),
        torch.tensor(batch["last"], dtype=torch.int32, device=dev),
    )


def oracle_weights(model):
    """The GPU model's weights as the oracle's fp32 host tensors, and its
    ``oracle.model.Shape``."""
    from oracle import model as om

    cfg = model.cfg
    f = lambda t: None if t is None else t.to("cpu", torch.float32)  # noqa: E731
    layers = [{"in_norm": f(L.in_norm), "post_norm": f(L.post_norm), "w_qkv": f(L.w_qkv), "b_qkv": f(L.b_qkv),
               "w_o": f(L.w_o), "w_gate_up": f(L.w_gate_up), "w_down": f(L.w_down)} for L in model.layers]
    embed = f(model.embed)
    lm = embed if model.lm_head is model.embed else f(model.lm_head)
    shape = om.Shape(cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                     cfg.intermediate_size, cfg.vocab_size, cfg.rms_norm_eps, cfg.rope_theta)
    return om.Weights(embed, lm, f(model.norm), layers), shape


# Bound on max |engine - oracle| / max |oracle| of a step's logits for the
# end-to-end config-2 check (24 layers, bf16 engine vs the fp32 oracle
# forward).  Measured drift of the bf16 engine: 1.5e-2 to 2.3e-2 per step;
# decode mistakes planted in the oracle (a RoPE / slot position off by one,
# the new token missing its own K / V) move the logits by 8e-2 to 2e-1
# (tests/test_oracle_model.py).
E2E_LOGIT_REL_BOUND = 4e-2
