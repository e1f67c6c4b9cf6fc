"""Write tests/golden/c1_decode.safetensors: the single-layer decode case.

Qwen2.5-0.5B head shape (14 Q heads, 2 KV heads, head_dim 64), B=4 requests
with contexts {17, 64, 203, 511}, page_size 16, pages taken as consecutive
slices of a seeded random permutation of a 128-page pool; q and the pool
~N(0,1) cast to bf16, seed 0; softmax scale 1/sqrt(64).  The expected output
is the CPU oracle's fp32 result.  Only the 51 pages in use are stored.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention as oatt  # noqa: E402

OUT = Path(__file__).resolve().parent / "c1_decode.safetensors"


def make():
    g = torch.Generator().manual_seed(0)
    lens = [17, 64, 203, 511]
    npages = [math.ceil(n / 16) for n in lens]
    perm = torch.randperm(128, generator=g)
    q = torch.randn(4, 14, 64, generator=g).to(torch.bfloat16)
    pool = torch.randn(128, 2, 16, 2, 64, generator=g).to(torch.bfloat16)
    indptr = [0]
    for n in npages:
        indptr.append(indptr[-1] + n)
    indices = perm[: indptr[-1]].to(torch.int32)
    last = [n - (p - 1) * 16 for n, p in zip(lens, npages)]
    out = oatt.decode(q, pool, indptr, indices.tolist(), last)
    return {
        "q": q,
        "page_ids": indices,
        "pages": pool[indices.long()].contiguous(),
        "indptr": torch.tensor(indptr, dtype=torch.int32),
        "last_page_len": torch.tensor(last, dtype=torch.int32),
        "out_fp32": out.contiguous(),
    }


if __name__ == "__main__":
    save_file(make(), str(OUT))
    print(OUT, OUT.stat().st_size)
