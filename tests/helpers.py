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
