"""Ragged paged prefill attention -- drop-in for
``flashinfer.prefill.BatchPrefillWithPagedKVCacheWrapper``.

Reference usage:
  construction  scheduler.py:530-534  (128 MB uint8 workspace, kv_layout="NHD")
  plan          scheduler.py:704-716  (qo_indptr, paged_kv_indptr, paged_kv_indices,
                                       paged_kv_last_page_len, causal=True)
  run           model.py:235          (q [total_q, H, D], kv_data of one layer)

``plan`` is a one-workgroup GPU kernel; it never synchronises.  Any number
of requests can share one call (``qo_indptr`` with B+1 entries); the
reference only ever passes one, and prefills requests one after another.
Any integer GQA group runs without Q-head padding.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from ._util import require_gpu, require_i32_vector, require_pool, require_rows, stream_of


class BatchPrefillWithPagedKVCacheWrapper:
    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD", **_unused):
        if kv_layout != "NHD":
            raise ValueError(f"kv_layout {kv_layout!r} not supported (NHD only)")
        require_gpu("float_workspace_buffer", float_workspace_buffer)
        self._ws = float_workspace_buffer
        self._ws_bytes = float_workspace_buffer.numel() * float_workspace_buffer.element_size()
        self._planned = False

    def plan(
        self,
        qo_indptr: torch.Tensor,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim_qk: int,
        page_size: int,
        head_dim_vo: int | None = None,
        custom_mask=None,
        packed_custom_mask=None,
        causal: bool = False,
        pos_encoding_mode: str = "NONE",
        window_left: int = -1,
        logits_soft_cap: float | None = None,
        sm_scale: float | None = None,
        q_data_type: torch.dtype = torch.bfloat16,
        kv_data_type: torch.dtype | None = None,
        max_total_q: int | None = None,
        **_unused,
    ) -> None:
        """``max_total_q`` bounds the query rows of the following ``run`` calls
        (default: the workspace's capacity); it only sizes the tile list."""
        if pos_encoding_mode != "NONE":
            raise ValueError("only pos_encoding_mode='NONE' is supported")
        if custom_mask is not None or packed_custom_mask is not None:
            raise ValueError("custom masks are not supported")
        if window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise ValueError("sliding windows and logit soft-capping are not supported")
        if head_dim_vo not in (None, head_dim_qk):
            raise ValueError("head_dim_vo must equal head_dim_qk")
        if q_data_type != torch.bfloat16 or (kv_data_type or q_data_type) != torch.bfloat16:
            raise ValueError("prefill attention is built for bf16")
        for n, t in (("qo_indptr", qo_indptr), ("paged_kv_indptr", paged_kv_indptr),
                     ("paged_kv_indices", paged_kv_indices), ("paged_kv_last_page_len", paged_kv_last_page_len)):
            require_i32_vector(n, t)
        batch = qo_indptr.numel() - 1
        if batch < 0 or paged_kv_indptr.numel() != batch + 1 or paged_kv_last_page_len.numel() < batch:
            raise ValueError("qo_indptr / paged_kv_indptr must have batch+1 entries")
        if num_qo_heads % num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        if max_total_q is None:
            max_total_q = self._capacity_rows(batch)
        _lib.call("mi_prefill_plan", self._ws.data_ptr(), self._ws_bytes, qo_indptr.data_ptr(),
                  paged_kv_indptr.data_ptr(), paged_kv_last_page_len.data_ptr(), batch, max_total_q,
                  num_qo_heads, num_kv_heads, head_dim_qk, page_size, stream_of(qo_indptr))
        self._batch, self._max_total_q = batch, max_total_q
        self._hq, self._hkv, self._d, self._ps = num_qo_heads, num_kv_heads, head_dim_qk, page_size
        self._indices = paged_kv_indices
        self._causal = bool(causal)
        self._scale = float(sm_scale) if sm_scale else 1.0 / math.sqrt(head_dim_qk)
        self._planned = True

    def _capacity_rows(self, batch: int) -> int:
        lo, hi = 0, 1 << 40
        lib = _lib.load()
        while lo < hi:  # largest total_q whose tile list fits the workspace
            mid = (lo + hi + 1) // 2
            if lib.mi_prefill_workspace_size(batch, mid) <= self._ws_bytes:
                lo = mid
            else:
                hi = mid - 1
        return lo

    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, *, out: torch.Tensor | None = None,
            return_lse: bool = False) -> torch.Tensor:
        if not self._planned:
            raise RuntimeError("run() called before plan()")
        if return_lse:
            raise ValueError("return_lse is not supported")
        num_pages, page_size, hkv, d = require_pool("paged_kv_cache", paged_kv_cache)
        if (page_size, hkv, d) != (self._ps, self._hkv, self._d):
            raise ValueError("pool geometry differs from plan")
        require_rows("q", q, self._hq, self._d)
        total_q = q.shape[0]
        if total_q > self._max_total_q:
            raise ValueError(f"q has {total_q} rows; plan was sized for {self._max_total_q}")
        if out is None:
            out = torch.empty_like(q, memory_format=torch.contiguous_format)
        else:
            require_rows("out", out, self._hq, self._d)
        _lib.call(
            "mi_prefill_run", self._ws.data_ptr(), self._ws_bytes, q.data_ptr(), q.stride(0), q.stride(1),
            paged_kv_cache.data_ptr(), num_pages, self._indices.data_ptr(), out.data_ptr(), out.stride(0),
            out.stride(1), self._batch, self._max_total_q, self._hq, self._hkv, self._d, self._ps,
            int(self._causal), self._scale, stream_of(q),
        )
        return out

    forward = run
