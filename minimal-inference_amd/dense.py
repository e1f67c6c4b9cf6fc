"""Fused dense-layer helpers: residual add + RMSNorm, SiLU-gated product.

``add_rms_norm(x, delta, weight, eps)`` stands for ``x = x + delta`` followed
by ``F.rms_norm(x, (H,), weight, eps)`` (DecoderLayer.forward,
model.py:324-344; RMSNorm, model.py:115-122); ``silu_mul(gate_up)`` for
``F.silu(gate) * up`` over the fused gate/up projection (MLP,
model.py:301-311).  Both run one HIP kernel (``mi_add_rms_norm`` /
``mi_silu_mul``); there is no torch fallback.
"""

from __future__ import annotations

import torch

from . import _lib
from ._util import require_dtype, require_gpu, stream_of


def _rows(name: str, t: torch.Tensor, width: int | None = None) -> None:
    require_gpu(name, t)
    require_dtype(name, t, torch.bfloat16)
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be [rows, width] with a contiguous last axis; got {tuple(t.shape)}")
    if width is not None and t.shape[1] != width:
        raise ValueError(f"{name} must have {width} columns; got {t.shape[1]}")


def add_rms_norm(x: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor, eps: float, *,
                 write_x: bool = True, norm: bool = True,
                 h_out: torch.Tensor | None = None) -> torch.Tensor | None:
    """In place: ``x += delta`` (bf16, when ``delta`` is given and ``write_x``);
    returns ``rms_norm(x + delta) * weight`` (or None when ``norm`` is false)."""
    rows, hidden = x.shape
    _rows("x", x)
    if delta is not None:
        _rows("delta", delta, hidden)
        if delta.shape[0] != rows:
            raise ValueError("delta rows differ from x")
    if norm:
        require_gpu("weight", weight)
        require_dtype("weight", weight, torch.bfloat16)
        if weight.dim() != 1 or weight.numel() != hidden or not weight.is_contiguous():
            raise ValueError(f"weight must be a contiguous [{hidden}] tensor")
        if h_out is None:
            h_out = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
        _rows("h_out", h_out, hidden)
    elif not (write_x and delta is not None):
        raise ValueError("nothing to do: neither the sum nor the norm is requested")
    xo = x if (write_x and delta is not None) else None
    _lib.call("mi_add_rms_norm", x.data_ptr(), x.stride(0),
              delta.data_ptr() if delta is not None else None, delta.stride(0) if delta is not None else 0,
              weight.data_ptr() if norm else None, xo.data_ptr() if xo is not None else None,
              xo.stride(0) if xo is not None else 0, h_out.data_ptr() if norm else None,
              h_out.stride(0) if norm else 0, rows, hidden, float(eps), stream_of(x))
    return h_out if norm else None


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate_up[:, :I]) * gate_up[:, I:]`` as one kernel; returns [rows, I]."""
    _rows("gate_up", gate_up)
    rows, width = gate_up.shape
    if width % 2:
        raise ValueError("gate_up must have an even number of columns")
    inter = width // 2
    if out is None:
        out = torch.empty(rows, inter, dtype=gate_up.dtype, device=gate_up.device)
    _rows("out", out, inter)
    _lib.call("mi_silu_mul", gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0), rows, inter,
              stream_of(gate_up))
    return out
