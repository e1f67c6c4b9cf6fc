"""Split-K paged decode attention -- drop-in for
``flashinfer.decode.BatchDecodeWithPagedKVCacheWrapper``.

Reference usage:
  construction  scheduler.py:535-539  (128 MB uint8 workspace, kv_layout="NHD")
  plan          scheduler.py:402-413, 905-916, 927-938
  run           model.py:235          (q [B, H, D], kv_data of one layer)

Differences that matter to a caller:
  * ``plan`` is a GPU kernel: it reads ``indptr`` / ``last_page_len`` on the
    device and never synchronises, so it can run every step outside a graph.
  * any integer GQA group 1..8 runs natively; the reference's zero-padding of
    Q heads to a power-of-two group (model.py:134-137, 226-243) is not needed.
  * ``run`` reads the work list ``plan`` left in the workspace and the page
    ids from the ``indices`` tensor given to ``plan`` (kept by reference, as
    the reference relies on, scheduler.py:898-899); ``plan`` also copies the
    first page ids of each split into the work list, so ``indices`` must not
    change between ``plan`` and ``run`` (the reference never does that).  The
    grid of ``run`` is fixed per (batch, heads, head_dim), so a graph captured
    once replays correctly after every later ``plan``.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from ._util import require_gpu, require_i32_vector, require_pool, require_rows, stream_of


class BatchDecodeWithPagedKVCacheWrapper:
    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, **_unused):
        if kv_layout != "NHD":
            raise ValueError(f"kv_layout {kv_layout!r} not supported (NHD only)")
        require_gpu("float_workspace_buffer", float_workspace_buffer)
        if not float_workspace_buffer.is_contiguous():
            raise ValueError("workspace must be contiguous")
        self._ws = float_workspace_buffer
        self._ws_bytes = float_workspace_buffer.numel() * float_workspace_buffer.element_size()
        self._planned = False

    # ------------------------------------------------------------------ plan
    def plan(
        self,
        indptr: torch.Tensor,
        indices: torch.Tensor,
        last_page_len: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        pos_encoding_mode: str = "NONE",
        window_left: int = -1,
        logits_soft_cap: float | None = None,
        q_data_type: torch.dtype = torch.bfloat16,
        kv_data_type: torch.dtype | None = None,
        data_type: torch.dtype | None = None,
        sm_scale: float | None = None,
        **_unused,
    ) -> None:
        if pos_encoding_mode != "NONE":
            raise ValueError("only pos_encoding_mode='NONE' is supported (RoPE is applied by the caller)")
        if window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise ValueError("sliding windows and logit soft-capping are not supported")
        kv_dtype = kv_data_type or data_type or q_data_type
        if q_data_type != torch.bfloat16 or kv_dtype != torch.bfloat16:
            raise ValueError("decode attention is built for bf16 q and kv")
        self._check_plan_args(indptr, indices, last_page_len, num_qo_heads, num_kv_heads)
        batch = indptr.numel() - 1
        _lib.call(
            "mi_decode_plan", self._ws.data_ptr(), self._ws_bytes, indptr.data_ptr(),
            indices.data_ptr(), last_page_len.data_ptr(), batch, num_qo_heads, num_kv_heads, head_dim, page_size, 0,
            stream_of(indptr),
        )
        self._adopt_plan(indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale)

    @staticmethod
    def _check_plan_args(indptr, indices, last_page_len, num_qo_heads: int, num_kv_heads: int) -> None:
        for n, t in (("indptr", indptr), ("indices", indices), ("last_page_len", last_page_len)):
            require_i32_vector(n, t)
        batch = indptr.numel() - 1
        if batch < 0 or last_page_len.numel() < batch:
            raise ValueError("indptr must have batch+1 entries and last_page_len batch entries")
        if num_qo_heads % num_kv_heads:
            raise ValueError(f"num_qo_heads {num_qo_heads} is not a multiple of num_kv_heads {num_kv_heads}")

    def _adopt_plan(self, indptr, indices, last_page_len, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                    page_size: int, sm_scale: float | None = None) -> None:
        """Record what run() needs of a plan that has been written into the
        workspace (by plan(), or by the page-table step that plans the batch
        it lays out in the same launch)."""
        self._batch = indptr.numel() - 1
        self._hq, self._hkv, self._d, self._ps = num_qo_heads, num_kv_heads, head_dim, page_size
        self._indices = indices
        self._indptr = indptr
        self._last_page_len = last_page_len
        self._scale = float(sm_scale) if sm_scale else 1.0 / math.sqrt(head_dim)
        self._planned = True

    @staticmethod
    def workspace_bytes(batch: int, num_qo_heads: int, num_kv_heads: int, head_dim: int) -> int:
        return int(_lib.load().mi_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim, 0))

    # ------------------------------------------------------------------ run
    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, *, out: torch.Tensor | None = None,
            return_lse: bool = False) -> torch.Tensor:
        if not self._planned:
            raise RuntimeError("run() called before plan()")
        if return_lse:
            raise ValueError("return_lse is not supported")
        num_pages, page_size, hkv, d = require_pool("paged_kv_cache", paged_kv_cache)
        if (page_size, hkv, d) != (self._ps, self._hkv, self._d):
            raise ValueError(f"pool geometry {(page_size, hkv, d)} differs from plan "
                             f"{(self._ps, self._hkv, self._d)}")
        require_rows("q", q, self._hq, self._d)
        if q.shape[0] != self._batch:
            raise ValueError(f"q has {q.shape[0]} rows, plan was for batch {self._batch}")
        if out is None:
            out = torch.empty_like(q, memory_format=torch.contiguous_format)
        else:
            require_rows("out", out, self._hq, self._d)
            if out.shape[0] != self._batch:
                raise ValueError("out batch differs from q")
        _lib.call(
            "mi_decode_run", self._ws.data_ptr(), self._ws_bytes, q.data_ptr(), q.stride(0), q.stride(1),
            paged_kv_cache.data_ptr(), num_pages, self._indices.data_ptr(), out.data_ptr(),
            out.stride(0), out.stride(1), self._batch, self._hq, self._hkv, self._d, self._ps,
            self._scale, 0, stream_of(q),
        )
        return out

    forward = run

    def run_rope_append(self, qkv: torch.Tensor, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
                        paged_kv_cache: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
        """The decode step's RoPE, K/V append and attention in one launch.

        Stands for ``rope_append_paged_kv_cache`` (the reference's RoPE on q
        and k, model.py:169-170, and ``append_paged_kv_cache``,
        model.py:203-216) followed by ``run`` (model.py:235) when every
        request of the plan appends exactly one token at its last position
        (position kv_len - 1, as in decode): ``qkv`` is ``[B, (Hq + 2 Hkv) *
        D]`` (q heads, k heads, v heads), request b is rotated with row
        kv_len_b - 1 (its decode position) of the bf16 ``[rows, D]`` tables,
        its rotated k and v go to slot ``last_page_len[b] - 1`` of its last
        page, and the result is the attention output ``[B, Hq, D]``.  Pool and
        output are bit-identical to the three-call sequence with rope positions
        kv_len - 1; ``qkv`` is not modified.
        """
        if not self._planned:
            raise RuntimeError("run_rope_append() called before plan()")
        num_pages, page_size, hkv, d = require_pool("paged_kv_cache", paged_kv_cache)
        if (page_size, hkv, d) != (self._ps, self._hkv, self._d):
            raise ValueError(f"pool geometry {(page_size, hkv, d)} differs from plan "
                             f"{(self._ps, self._hkv, self._d)}")
        require_gpu("qkv", qkv)
        if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.stride(1) != 1:
            raise ValueError("qkv must be a [B, (Hq + 2 Hkv) * D] bf16 tensor with contiguous rows")
        if qkv.shape != (self._batch, (self._hq + 2 * self._hkv) * d):
            raise ValueError(f"qkv is {tuple(qkv.shape)}, the plan needs "
                             f"({self._batch}, {(self._hq + 2 * self._hkv) * d})")
        for name, tab in (("cos_cache", cos_cache), ("sin_cache", sin_cache)):
            require_gpu(name, tab)
            if tab.dtype != torch.bfloat16 or tab.dim() != 2 or tab.shape[1] != d or not tab.is_contiguous():
                raise ValueError(f"{name} must be a contiguous [rows, {d}] bf16 table")
        if cos_cache.shape != sin_cache.shape:
            raise ValueError("cos_cache and sin_cache differ in shape")
        if out is None:
            out = torch.empty(self._batch, self._hq, d, dtype=qkv.dtype, device=qkv.device)
        else:
            require_rows("out", out, self._hq, d)
            if out.shape[0] != self._batch:
                raise ValueError("out batch differs from the plan")
        _lib.call(
            "mi_decode_rope_append_run", self._ws.data_ptr(), self._ws_bytes, qkv.data_ptr(), qkv.stride(0),
            cos_cache.data_ptr(), sin_cache.data_ptr(), cos_cache.shape[0],
            paged_kv_cache.data_ptr(), num_pages, self._indices.data_ptr(), out.data_ptr(), out.stride(0),
            out.stride(1), self._batch, self._hq, self._hkv, d, self._ps, self._scale, 0, stream_of(qkv),
        )
        return out
