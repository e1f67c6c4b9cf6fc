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

The single-request ``sample`` (scheduler.py:310-316) differs in two ways,
restated by ``sample_distribution``:

* the temperature stays a Python float: ``logits[0, -1] / temperature`` is a
  bf16 tensor divided by a scalar, which PyTorch's GPU kernel computes as the
  product with the scalar's fp32 reciprocal, rounded to bf16 (313);
* ``F.softmax(scaled, dim=-1)`` has no dtype argument, so the probabilities
  are rounded to bf16 (fp32 arithmetic inside) and ``multinomial`` draws in
  proportion to those bf16 values (314-315).

top-p is an extension beyond the reference: the nucleus is the set of tokens
whose probability is at least the smallest probability p* such that the mass
of tokens with probability >= p* reaches top_p (ties at p* are kept).

Pinning (tests/test_oracle_sampling.py): greedy against numpy argmax and hand
cases (ties, NaN); temperature quantisation against known bf16 values; the
nucleus against a sort-based brute force and hand-derived small cases;
``sample_distribution`` against hand-derived bf16 probabilities and a case
where the reciprocal product and the quotient round apart (and, on the GPU,
tests/test_gpu_sampler.py checks the scalar division and the bf16 softmax
against torch's own GPU kernels).
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


def scalar_scaled_logits(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """``logits / temperature`` for a bf16 tensor and a Python-float
    temperature (scheduler.py:313): the fp32 product with the fp32
    reciprocal of the temperature, rounded to bf16."""
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(temperature, dtype=torch.float32)
    return (logits.to(torch.bfloat16).float() * inv).to(torch.bfloat16)


def sample_distribution(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """Distribution of ``sample(logits [1, S, V], temperature)`` over the
    vocabulary for one row ``logits`` [V] (scheduler.py:310-316): one-hot at
    the first argmax when temperature <= 0; else softmax of the bf16 scaled
    logits rounded to bf16, normalised as multinomial does (float64)."""
    row = logits.to(torch.bfloat16)
    if temperature <= 0:
        out = torch.zeros(row.shape[-1], dtype=torch.float64)
        out[int(greedy(row))] = 1.0
        return out
    p = torch.softmax(scalar_scaled_logits(row, temperature).float(), dim=-1).to(torch.bfloat16).double()
    return p / p.sum()
