"""Rotary position embedding -- oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates the reference's RoPE in plain torch on the CPU:

* ``tables`` -- precompute_rope (model.py:79-89): inv_freq = 1 / theta^(2i/d),
  freqs = outer(t, inv_freq), emb = cat(freqs, freqs); cos / sin of emb in
  fp32, then cast to the model dtype as the server does (server.py:251).
* ``apply`` -- apply_rotary_emb (model.py:92-107): rotate-half,
  ``x * cos + cat(-x2, x1) * sin`` evaluated as three bf16 torch ops (each
  rounds its fp32 result to bf16), cos / sin broadcast over heads.

Pinning (tests/test_oracle_rope.py): position 0 is the identity; the pair
(j, j + d/2) is a plane rotation by angle p * inv_freq[j] (float64 closed
form, within bf16 rounding); rotations compose (p then q equals p + q within
rounding); and the bf16 rounding order is checked against an explicit
element-wise evaluation of the three roundings, so a fused kernel that keeps
fp32 between the ops (a plausible mistake) fails.
"""

from __future__ import annotations

import torch


def tables(head_dim: int, max_len: int, theta: float, dtype=torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin ``[max_len, head_dim]`` (model.py:79-89), cast to ``dtype``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    t = torch.arange(max_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x ``[T, H, D]``, cos / sin ``[T, D]`` (already gathered by position)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    rotated = torch.cat((-x2, x1), dim=-1)
    return x * cos.unsqueeze(1) + rotated * sin.unsqueeze(1)


def rope_append(qkv: torch.Tensor, hq: int, hkv: int, rope_pos: list[int], cos: torch.Tensor, sin: torch.Tensor,
                pool: torch.Tensor, indptr: list[int], indices: list[int], batch_indices: list[int],
                positions: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
    """The unfused sequence the fused kernel stands for: rotate q and k of
    every row of ``qkv`` ``[T, (hq + 2 hkv) * D]`` with table row
    ``rope_pos[i]`` (clamped to the table), then append k / v into a copy of
    ``pool`` (oracle.paging.append placement).  Returns (q, new pool)."""
    from .paging import append

    t = qkv.shape[0]
    d = pool.shape[-1]
    rows = [min(max(p, 0), cos.shape[0] - 1) for p in rope_pos]
    c, s = cos[rows], sin[rows]
    q = apply(qkv[:, : hq * d].view(t, hq, d), c, s)
    k = apply(qkv[:, hq * d: (hq + hkv) * d].view(t, hkv, d), c, s)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    return q, append(pool, k, v, batch_indices, positions, indices, indptr)
