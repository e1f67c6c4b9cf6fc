"""CPU: pin the sampling oracle.

Greedy against numpy's argmax (first index on ties); the bf16 temperature
quantisation against known bf16 values; the distribution against the closed
form exp(s)/sum exp(s); the top-p nucleus against a sort-based brute force.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import sampling as osmp


def test_greedy_first_index_on_ties():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0]]).to(torch.bfloat16)
    assert osmp.greedy(x).tolist() == [1, 0]
    r = torch.randn(5, 1000).to(torch.bfloat16)
    assert osmp.greedy(r).tolist() == np.argmax(r.float().numpy(), axis=-1).tolist()


def test_temperature_rounds_to_bf16():
    t = osmp.quantized_temperature([0.7, 1.0, 0.9, 0.0])
    assert t.float().tolist() == [0.69921875, 1.0, 0.8984375, 0.0]


def test_distribution_closed_form():
    logits = torch.tensor([[0.0, 1.0, 2.0, -1.0]]).to(torch.bfloat16)
    p = osmp.distribution(logits, [1.0])[0].double()
    e = np.exp(np.array([0.0, 1.0, 2.0, -1.0]))
    assert np.allclose(p.numpy(), e / e.sum(), atol=1e-6)
    # temperature 0.7 quantised to 0.69921875, quotient rounded to bf16
    p7 = osmp.distribution(logits, [0.7])[0].double()
    s = (torch.tensor([0.0, 1.0, 2.0, -1.0]) / 0.69921875).to(torch.bfloat16).double().numpy()
    e = np.exp(s - s.max())
    assert np.allclose(p7.numpy(), e / e.sum(), atol=1e-6)


def _nucleus_bruteforce(p: np.ndarray, top_p: float) -> np.ndarray:
    order = np.argsort(-p, kind="stable")
    keep = np.zeros_like(p, dtype=bool)
    mass = 0.0
    i = 0
    while i < len(order):
        v = p[order[i]]
        ties = [j for j in order[i:] if p[j] == v]
        if mass >= top_p:
            break
        for j in ties:
            keep[j] = True
        mass += v * len(ties)
        i += len(ties)
    return keep


def test_top_p_matches_sort_bruteforce():
    rng = np.random.default_rng(0)
    for trial in range(30):
        v = int(rng.integers(2, 60))
        logits = torch.tensor(rng.normal(size=(1, v)) * 2).to(torch.bfloat16)
        top_p = float(rng.uniform(0.05, 0.99))
        base = osmp.distribution(logits, [1.0])[0].double().numpy()
        got = osmp.distribution(logits, [1.0], [top_p])[0].double().numpy()
        keep = _nucleus_bruteforce(base, top_p)
        assert np.array_equal(got > 0, keep)
        assert np.allclose(got[keep], base[keep] / base[keep].sum(), atol=1e-6)


def test_top_p_hand_case():
    p = torch.log(torch.tensor([[0.5, 0.3, 0.15, 0.05]]))
    logits = p.to(torch.bfloat16)
    got = osmp.distribution(logits, [1.0], [0.7])[0]
    assert (got > 0).tolist() == [True, True, False, False]
    got = osmp.distribution(logits, [1.0], [0.5])[0]
    assert (got > 0).tolist() == [True, False, False, False]


def test_sample_keeps_the_float_temperature():
    """sample() divides by the Python float (0.7 stays 0.7), sample_batch by
    its bf16 rounding 0.69921875: the scaled logits differ for some inputs."""
    x = torch.arange(0x3F80, 0x4100, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)  # [1, 8)
    a = osmp.scalar_scaled_logits(x, 0.7)
    b = osmp.scaled_logits(x.unsqueeze(0), [0.7])[0]
    want = (x.double() / 0.7).float().to(torch.bfloat16)  # float64 quotient: same bf16 rounding here
    assert torch.equal(a, want)
    assert int((a != b).sum()) > 0


def test_sample_reciprocal_product_rounding():
    """Near the bottom of the fp32 normal range the product with the fp32
    reciprocal of 0.3 and the quotient round to different bf16 values; the
    restatement takes the product."""
    x = torch.tensor([2.1765012589443917e-38]).to(torch.bfloat16)
    inv = torch.tensor(1.0) / torch.tensor(0.3)
    assert float(osmp.scalar_scaled_logits(x, 0.3)[0]) == float((x.float() * inv).to(torch.bfloat16)[0])
    assert float(osmp.scalar_scaled_logits(x, 0.3)[0]) != float((x.float() / 0.3).to(torch.bfloat16)[0])


def test_sample_distribution_bf16_probabilities():
    """Logits [0, bf16(ln 2)] at temperature 1: fp32 softmax (0.33374,
    0.66626) rounds to bf16 171 * 2^-9 and 171 * 2^-8, which multinomial
    normalises to exactly 1/3 and 2/3."""
    x = torch.tensor([0.0, 0.69140625]).to(torch.bfloat16)
    p = osmp.sample_distribution(x, 1.0)
    assert p.tolist() == [1 / 3, 2 / 3]
    assert osmp.sample_distribution(x, 0.0).tolist() == [0.0, 1.0]
    assert osmp.sample_distribution(torch.tensor([2.0, 2.0, 1.0]), -1.0).tolist() == [1.0, 0.0, 0.0]
