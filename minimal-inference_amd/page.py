"""Paged KV append -- the drop-in for ``flashinfer.page.append_paged_kv_cache``.

Reference call: model.py:207-216 passes, positionally, ``append_key,
append_value, batch_indices, positions, paged_kv_cache, kv_indices,
kv_indptr, kv_last_page_len`` with an NHD pool
(scheduler.py:195-202: ``[max_pages, 2, page_size, kv_heads, head_dim]``).
"""

from __future__ import annotations

import torch

from . import _lib
from ._util import require_gpu, require_i32_vector, require_pool, require_rows, stream_of


def append_paged_kv_cache(
    append_key: torch.Tensor,
    append_value: torch.Tensor,
    batch_indices: torch.Tensor,
    positions: torch.Tensor,
    paged_kv_cache: torch.Tensor,
    kv_indices: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_last_page_len: torch.Tensor,
    kv_layout: str = "NHD",
) -> None:
    """Write K/V rows ``[T, kv_heads, head_dim]`` into their page slots.

    Token i goes to page ``kv_indices[kv_indptr[b] + p // page_size]``, slot
    ``p % page_size`` with ``b = batch_indices[i]``, ``p = positions[i]``.
    Tokens whose slot lies outside request b's page list are not written.
    Runs asynchronously on the current stream; safe under graph capture.
    """
    if kv_layout != "NHD":
        raise ValueError(f"kv_layout {kv_layout!r} not supported (NHD only)")
    num_pages, page_size, hkv, d = require_pool("paged_kv_cache", paged_kv_cache)
    require_rows("append_key", append_key, hkv, d)
    require_rows("append_value", append_value, hkv, d)
    if append_value.shape[0] != append_key.shape[0]:
        raise ValueError("append_key and append_value disagree on the token count")
    for n, t in (("batch_indices", batch_indices), ("positions", positions), ("kv_indices", kv_indices),
                 ("kv_indptr", kv_indptr), ("kv_last_page_len", kv_last_page_len)):
        require_i32_vector(n, t)
    t_count = append_key.shape[0]
    if batch_indices.numel() != t_count or positions.numel() != t_count:
        raise ValueError("batch_indices / positions must have one entry per appended token")
    batch = kv_indptr.numel() - 1
    if batch < 0:
        raise ValueError("kv_indptr must have batch_size + 1 entries")
    for name, t in (("append_key", append_key), ("append_value", append_value)):
        if t.device != paged_kv_cache.device:
            raise ValueError(f"{name} is on {t.device}, pool on {paged_kv_cache.device}")
    require_gpu("kv_indices", kv_indices)
    _lib.call(
        "mi_paged_kv_append",
        append_key.data_ptr(), append_key.stride(0), append_key.stride(1),
        append_value.data_ptr(), append_value.stride(0), append_value.stride(1),
        batch_indices.data_ptr(), positions.data_ptr(), t_count,
        paged_kv_cache.data_ptr(), num_pages,
        kv_indices.data_ptr(), kv_indptr.data_ptr(), kv_last_page_len.data_ptr(),
        batch, hkv, d, page_size, stream_of(paged_kv_cache),
    )
