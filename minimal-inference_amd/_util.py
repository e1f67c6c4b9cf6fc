"""Argument checks and stream plumbing shared by the wrappers."""

from __future__ import annotations

import torch


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on ``t``'s device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU (got {t.device}); there is no CPU path")


def require_dtype(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")


def require_i32_vector(name: str, t: torch.Tensor) -> None:
    require_gpu(name, t)
    require_dtype(name, t, torch.int32)
    if t.dim() != 1 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous 1-D int32 tensor (got shape {tuple(t.shape)})")


def require_pool(name: str, pool: torch.Tensor) -> tuple[int, int, int, int]:
    """Validate an NHD pool [pages, 2, page_size, kv_heads, head_dim] bf16."""
    require_gpu(name, pool)
    require_dtype(name, pool, torch.bfloat16)
    if pool.dim() != 5 or pool.shape[1] != 2:
        raise ValueError(f"{name} must be [num_pages, 2, page_size, num_kv_heads, head_dim] "
                         f"(NHD); got {tuple(pool.shape)}")
    if not pool.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return tuple(int(x) for x in (pool.shape[0], pool.shape[2], pool.shape[3], pool.shape[4]))


def require_rows(name: str, t: torch.Tensor, heads: int, head_dim: int) -> None:
    """[N, heads, head_dim] bf16 with head_dim contiguous."""
    require_gpu(name, t)
    require_dtype(name, t, torch.bfloat16)
    if t.dim() != 3 or t.shape[1] != heads or t.shape[2] != head_dim:
        raise ValueError(f"{name} must be [N, {heads}, {head_dim}]; got {tuple(t.shape)}")
    if t.stride(2) != 1:
        raise ValueError(f"{name} must have a contiguous last axis")
