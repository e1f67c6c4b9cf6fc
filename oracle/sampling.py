"""Batched sampler semantics -- oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates sample_batch (scheduler.py:319-343):

* the temperature tensor has the logits dtype (bf16), so 0.7 becomes
  0.69921875 (327); rows with temperature <= 0 are greedy (328);
* ``scaled = logits / clamp(temps, 1e-6)`` is computed on bf16 tensors, i.e.
  an fp32 division rounded to bf16 (331-332);
* ``probs = softmax(scaled, dtype=float32)`` (333), one multinomial draw (336);
* greedy rows take ``argmax(logits)`` -- the first index among equal maxima
  (339-341).

top-p is an extension beyond the reference: the nucleus is the set of tokens
whose probability is at least the smallest probability p* such that the mass
of tokens with probability >= p* reaches top_p (ties at p* are kept).

Pinning (tests/test_oracle_sampling.py): greedy against numpy argmax and hand
cases (ties, NaN); temperature quantisation against known bf16 values; the
nucleus against a sort-based brute force and hand-derived small cases.
"""

from __future__ import annotations

import torch


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """argmax over the last axis, first index among ties (scheduler.py:340)."""
    return logits.argmax(dim=-1)


def quantized_temperature(temperatures: list[float]) -> torch.Tensor:
    """temperatures as the reference holds them: a bf16 tensor (327)."""
    return torch.tensor(temperatures, dtype=torch.bfloat16)


def scaled_logits(logits: torch.Tensor, temperatures: list[float]) -> torch.Tensor:
    """bf16 logits [B, V] / clamp(bf16 temps, 1e-6) in bf16 (331-332)."""
    temps = quantized_temperature(temperatures).clamp(min=1e-6).unsqueeze(1)
    return logits.to(torch.bfloat16) / temps


def distribution(logits: torch.Tensor, temperatures: list[float],
                 top_p: list[float] | None = None) -> torch.Tensor:
    """fp32 sampling distribution per row [B, V] (softmax at 333, + top-p)."""
    probs = torch.softmax(scaled_logits(logits, temperatures).float(), dim=-1)
    if top_p is None:
        return probs
    out = probs.clone()
    for b, p in enumerate(top_p):
        if p >= 1.0:
            continue
        row = probs[b]
        # keep token i iff mass of tokens with prob >= prob_i ... resolved per
        # distinct value: the kept set is {i : mass(probs > probs_i) < p}
        vals = torch.unique(row, sorted=True).flip(0)
        above = 0.0
        thresh = vals[-1]
        for val in vals.tolist():
            if above >= p:
                break
            thresh = val
            above += float(row[row == val].sum())
        keep = row >= thresh
        out[b] = torch.where(keep, row, torch.zeros_like(row))
        out[b] /= out[b].sum()
    return out
