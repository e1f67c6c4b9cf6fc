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


def rope_append_paged_kv_cache(
    qkv: torch.Tensor,
    num_qo_heads: int,
    num_kv_heads: int,
    rope_positions: torch.Tensor,
    cos_cache: torch.Tensor,
    sin_cache: torch.Tensor,
    batch_indices: torch.Tensor,
    positions: torch.Tensor,
    paged_kv_cache: torch.Tensor,
    kv_indices: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_last_page_len: torch.Tensor,
    q_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Rotate q and k of the fused projection rows and append k / v, in one launch.

    Stands for the reference's ``apply_rotary_emb`` on q and k
    (model.py:92-107, 169-170) followed by ``append_paged_kv_cache``
    (model.py:203-216), with bit-identical results: ``cos_cache`` /
    ``sin_cache`` are the bf16 ``[max_positions, head_dim]`` tables and token
    i uses row ``rope_positions[i]``.  ``qkv`` is ``[T, (Hq + 2 Hkv) * D]``
    (q heads, k heads, v heads).  Returns the rotated q as ``[T, Hq, D]``:
    ``q_out`` if given, else a view of ``qkv``'s q columns rotated in place.
    """
    num_pages, page_size, hkv, d = require_pool("paged_kv_cache", paged_kv_cache)
    if num_kv_heads != hkv:
        raise ValueError(f"num_kv_heads {num_kv_heads} != pool's {hkv}")
    require_gpu("qkv", qkv)
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a [T, (Hq + 2 Hkv) * D] bf16 tensor with contiguous rows")
    if qkv.shape[1] != (num_qo_heads + 2 * num_kv_heads) * d:
        raise ValueError(f"qkv has {qkv.shape[1]} columns, expected (Hq + 2 Hkv) * D = "
                         f"{(num_qo_heads + 2 * num_kv_heads) * d}")
    for name, tab in (("cos_cache", cos_cache), ("sin_cache", sin_cache)):
        require_gpu(name, tab)
        if tab.dtype != torch.bfloat16 or tab.dim() != 2 or tab.shape[1] != d or not tab.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [rows, {d}] bf16 table")
    if cos_cache.shape != sin_cache.shape:
        raise ValueError("cos_cache and sin_cache differ in shape")
    for n, t in (("rope_positions", rope_positions), ("batch_indices", batch_indices), ("positions", positions),
                 ("kv_indices", kv_indices), ("kv_indptr", kv_indptr), ("kv_last_page_len", kv_last_page_len)):
        require_i32_vector(n, t)
    t_count = qkv.shape[0]
    for n, t in (("rope_positions", rope_positions), ("batch_indices", batch_indices), ("positions", positions)):
        if t.numel() != t_count:
            raise ValueError(f"{n} must have one entry per token ({t_count})")
    if q_out is None:
        q_out = qkv[:, : num_qo_heads * d].view(t_count, num_qo_heads, d)
    else:
        require_rows("q_out", q_out, num_qo_heads, d)
        if q_out.shape[0] != t_count:
            raise ValueError("q_out must have one row per token")
    batch = kv_indptr.numel() - 1
    _lib.call(
        "mi_rope_append",
        qkv.data_ptr(), qkv.stride(0), rope_positions.data_ptr(), cos_cache.data_ptr(), sin_cache.data_ptr(),
        cos_cache.shape[0], q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        batch_indices.data_ptr(), positions.data_ptr(), t_count,
        paged_kv_cache.data_ptr(), num_pages, kv_indices.data_ptr(), kv_indptr.data_ptr(),
        kv_last_page_len.data_ptr(), batch, num_qo_heads, num_kv_heads, d, page_size,
        stream_of(paged_kv_cache),
    )
    return q_out
