"""GPU parity: fused sampler.

Greedy ids are bit-exact against torch.argmax on the same bf16 logits.
Temperature / top-p draws are checked statistically (chi-square against the
oracle's fp32 distribution, p > 1e-4) and by support (every draw lies in the
top-p nucleus).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import sampling as osmp

pytestmark = pytest.mark.gpu


def _sampler(dev, n, seed=123):
    from minimal_inference_amd.sampling import Sampler

    return Sampler(dev, n, seed=seed)


@pytest.mark.parametrize("V", [32768, 151936, 1000, 7])
def test_greedy_bit_exact(dev, V):
    g = torch.Generator().manual_seed(V)
    logits = torch.randn(16, V, generator=g).to(torch.bfloat16)
    logits[3, :] = 0.0            # all ties -> index 0
    logits[4, V // 2] = 100.0     # clear max
    logits[5, 1] = logits[5, V - 1] = 50.0  # tie between two maxima -> first
    s = _sampler(dev, 16)
    s.set_params([0.0] * 16)
    got = s.sample(logits.to(dev)).cpu()
    assert torch.equal(got, osmp.greedy(logits))


def test_greedy_nan_and_negative_zero(dev):
    logits = torch.full((3, 100), -1.0).to(torch.bfloat16)
    logits[0, 40] = float("nan")
    logits[0, 90] = 5.0
    logits[1, 10] = -0.0
    logits[1, 20] = 0.0
    logits[2, :] = float("-inf")
    logits[2, 7] = float("nan")
    s = _sampler(dev, 3)
    s.set_params([0.0, -1.0, 0.0])
    got = s.sample(logits.to(dev)).cpu()
    assert torch.equal(got, logits.argmax(dim=-1))


def test_sample_batch_api_mixed_rows(dev):
    from minimal_inference_amd.sampling import sample_batch

    g = torch.Generator().manual_seed(1)
    logits = torch.randn(8, 1, 5000, generator=g).to(torch.bfloat16)
    temps = [0.0, 0.7, 0.0, 1.0, 0.0, 0.7, 0.0, 0.0]
    ids = sample_batch(logits.to(dev), temps)
    want = logits[:, -1].argmax(dim=-1).tolist()
    for i, t in enumerate(temps):
        if t <= 0:
            assert ids[i] == want[i]
        assert 0 <= ids[i] < 5000


def _chi2_ok(counts: np.ndarray, probs: np.ndarray, n: int) -> bool:
    from scipy.stats import chi2

    exp = probs * n
    keep = exp >= 5
    stat = float((((counts - exp) ** 2) / np.maximum(exp, 1e-12))[keep].sum())
    rest_o, rest_e = counts[~keep].sum(), exp[~keep].sum()
    dof = int(keep.sum()) - 1
    if rest_e > 0:
        stat += (rest_o - rest_e) ** 2 / max(rest_e, 1e-12)
        dof += 1
    return chi2.sf(stat, max(dof, 1)) > 1e-4


@pytest.mark.parametrize("temp,top_p", [(1.0, None), (0.7, None), (0.7, 0.9), (1.3, 0.5),
                                        # extremes: a near-greedy temperature, a nucleus of the top
                                        # token alone, a flat high-temperature nucleus
                                        (0.2, None), (1.0, 0.001), (2.5, 0.95)])
def test_distribution_matches_oracle(dev, temp, top_p):
    V, rows, calls = 64, 2048, 8
    g = torch.Generator().manual_seed(int(temp * 10) + (0 if top_p is None else 7))
    base = (torch.randn(V, generator=g) * 1.5).to(torch.bfloat16)
    logits = base.unsqueeze(0).repeat(rows, 1).contiguous()
    s = _sampler(dev, rows, seed=99)
    s.set_params([temp] * rows, None if top_p is None else [top_p] * rows)
    counts = np.zeros(V, dtype=np.int64)
    ld = logits.to(dev)
    for _ in range(calls):
        ids = s.sample(ld, use_top_p=top_p is not None).cpu().numpy()
        counts += np.bincount(ids, minlength=V)
    probs = osmp.distribution(base.unsqueeze(0), [temp], None if top_p is None else [top_p])[0].double().numpy()
    assert counts[probs == 0].sum() == 0, "drew a token outside the nucleus"
    assert _chi2_ok(counts, probs, rows * calls)


def test_top_p_support_large_vocab(dev):
    V, rows = 151936, 64
    g = torch.Generator().manual_seed(5)
    logits = (torch.randn(rows, V, generator=g) * 3).to(torch.bfloat16)
    s = _sampler(dev, rows, seed=5)
    s.set_params([0.7] * rows, [0.9] * rows)
    ids = s.sample(logits.to(dev)).cpu()
    probs = osmp.distribution(logits, [0.7] * rows, [0.9] * rows)
    for r in range(rows):
        assert probs[r, ids[r]] > 0


def test_rng_advances_between_calls(dev):
    V, rows = 1000, 256
    logits = torch.zeros(rows, V).to(torch.bfloat16)
    s = _sampler(dev, rows, seed=7)
    s.set_params([1.0] * rows)
    a = s.sample(logits.to(dev)).cpu().clone()
    b = s.sample(logits.to(dev)).cpu().clone()
    assert not torch.equal(a, b)
    # uniform logits: draws cover many ids
    assert len(set(a.tolist())) > 150


def test_top_p_boundary_inside_one_bin(dev):
    """Every scaled logit in [1, 1.5): all keys share one of the sampler's
    1,024 coarse bins, so the nucleus boundary is resolved among that bin's
    64 keys; draws must follow the oracle's nucleus distribution."""
    V, rows, calls = 256, 2048, 8
    g = torch.Generator().manual_seed(21)
    base = (1.0 + 0.5 * torch.rand(V, generator=g)).to(torch.bfloat16)
    logits = base.unsqueeze(0).repeat(rows, 1).contiguous()
    s = _sampler(dev, rows, seed=17)
    s.set_params([1.0] * rows, [0.5] * rows)
    counts = np.zeros(V, dtype=np.int64)
    ld = logits.to(dev)
    for _ in range(calls):
        counts += np.bincount(s.sample(ld).cpu().numpy(), minlength=V)
    probs = osmp.distribution(base.unsqueeze(0), [1.0], [0.5])[0].double().numpy()
    assert counts[probs == 0].sum() == 0, "drew a token outside the nucleus"
    assert 0 < (probs > 0).sum() < V
    assert _chi2_ok(counts, probs, rows * calls)


def _order_keys(x: torch.Tensor) -> torch.Tensor:
    """The 16-bit order keys of bf16 values (larger value, larger key); the
    sampler's coarse bins are key >> 6."""
    b = x.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    return torch.where((b & 0x8000) != 0, (~b) & 0xFFFF, b | 0x8000)


def _multichunk_logits(V, temp, seed, sigma=0.8, ratio=2.0, top=5 * 4096 + 17):
    """One token at logit 0 (chunk 5) and V - 1 background logits
    N(-a, sigma) with ``a`` set so that the background holds ``ratio`` times
    the top token's mass after scaling by 1 / temp: every 4,096-token chunk
    carries mass, the top token's chunk max lies more than 2^8 above every
    other chunk's max (so the per-chunk rescale of the coarse bins matters),
    and the nucleus boundary falls inside the background, in a bin whose
    tokens come from every chunk."""
    g = torch.Generator().manual_seed(seed)
    a = temp * math.log(V / ratio) + sigma * sigma / (2 * temp)
    x = -a + sigma * torch.randn(V, generator=g)
    x[top] = 0.0
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("V", [32768, 152064])
@pytest.mark.parametrize("temp,top_p", [(0.7, 0.9), (1.3, 0.5)])
def test_distribution_across_chunks(dev, V, temp, top_p):
    """Vocabularies of 8 and 38 chunks (the configs' 32,768 and 152,064): the
    cross-chunk path -- per-chunk bins rescaled by 2^(chunk max - row max),
    the merged-bin boundary search, the race over every chunk -- gives draws
    that follow the oracle's nucleus distribution.  Checked by chi-square per
    chunk (the rescale), per distinct scaled value (the weighting and the
    boundary key, whose tied tokens sit in every chunk), and by support."""
    C = 4096
    base = _multichunk_logits(V, temp, seed=V + int(temp * 10))
    probs = osmp.distribution(base.unsqueeze(0), [temp], [top_p])[0].double()
    scaled = osmp.scaled_logits(base.unsqueeze(0), [temp])[0]
    keys = _order_keys(scaled)
    nchunks = (V + C - 1) // C
    # the workload has the properties the test is about
    cmax = torch.stack([scaled[c * C:(c + 1) * C].float().max() for c in range(nchunks)]) * math.log2(math.e)
    top2 = cmax.sort(descending=True).values[:2]
    assert float(top2[0] - top2[1]) > 8.0, "chunk maxima must lie more than 2^8 apart"
    kept = probs > 0
    kmin = int(keys[kept].min())
    in_bin = kept & ((keys >> 6) == (kmin >> 6))
    assert torch.unique(torch.nonzero(in_bin)[:, 0] // C).numel() == nchunks, "boundary bin spans every chunk"
    assert int((keys == kmin).sum()) > 100 and 0 < int(kept.sum()) < V

    rows, calls = 4096, 32
    ld = base.to(dev).unsqueeze(0).expand(rows, V).contiguous()
    s = _sampler(dev, rows, seed=V + 11)
    s.set_params([temp] * rows, [top_p] * rows)
    counts = torch.zeros(V, dtype=torch.int64)
    for _ in range(calls):
        counts += torch.bincount(s.sample(ld).cpu(), minlength=V)
    n = rows * calls
    assert int(counts[~kept].sum()) == 0, "drew a token outside the nucleus"
    chunk_of = torch.arange(V) // C
    by_chunk = torch.zeros(nchunks, dtype=torch.int64).index_add_(0, chunk_of, counts)
    p_chunk = torch.zeros(nchunks, dtype=torch.float64).index_add_(0, chunk_of, probs)
    assert _chi2_ok(by_chunk.numpy(), p_chunk.numpy(), n), (by_chunk.tolist(), (p_chunk * n).round().tolist())
    uniq, inv = torch.unique(keys, return_inverse=True)
    by_key = torch.zeros(uniq.numel(), dtype=torch.int64).index_add_(0, inv, counts)
    p_key = torch.zeros(uniq.numel(), dtype=torch.float64).index_add_(0, inv, probs)
    assert _chi2_ok(by_key.numpy(), p_key.numpy(), n)


def test_batch_sizes_alternate_on_one_workspace(dev):
    """Calls with different batch sizes share the sampler's workspace (its
    counters sit at fixed offsets): greedy rows stay bit-exact throughout."""
    V = 40000
    g = torch.Generator().manual_seed(8)
    s = _sampler(dev, 48)
    for n in (48, 3, 17, 48, 1):
        logits = torch.randn(n, V, generator=g).to(torch.bfloat16)
        temps = [0.0 if i % 2 == 0 else 0.7 for i in range(n)]
        s.set_params(temps, [1.0 if i % 4 == 1 else 0.9 for i in range(n)])
        got = s.sample(logits.to(dev)).cpu()
        want = osmp.greedy(logits)
        for i in range(n):
            if temps[i] == 0.0:
                assert got[i] == want[i], (n, i)
            else:
                assert 0 <= got[i] < V


def test_unaligned_rows_and_partial_last_chunk(dev):
    """Rows at an odd element stride (2-byte aligned only: the per-token load
    path) and a vocabulary that ends inside a 4-token group and inside its
    last 4,096-token chunk: greedy ids stay bit-exact, draws stay inside the
    nucleus."""
    V, rows = 9001, 24
    g = torch.Generator().manual_seed(33)
    full = (torch.randn(rows, V + 1, generator=g) * 2).to(torch.bfloat16)
    logits = full[:, :V].contiguous()
    temps = [0.0 if i % 3 == 0 else 0.8 for i in range(rows)]
    s = _sampler(dev, rows, seed=3)
    s.set_params(temps, [0.9] * rows)
    view = full.to(dev)[:, :V]
    assert view.stride(0) == V + 1
    got = s.sample(view).cpu()
    want = osmp.greedy(logits)
    sampled = [i for i in range(rows) if temps[i] > 0]
    probs = osmp.distribution(logits[sampled], [temps[i] for i in sampled], [0.9] * len(sampled))
    for i in range(rows):
        if temps[i] == 0.0:
            assert got[i] == want[i], i
    for k, i in enumerate(sampled):
        assert probs[k, got[i]] > 0, (i, int(got[i]))


def test_largest_vocabulary_and_one_past_it(dev):
    """1,048,576 tokens (256 chunks of 4,096, the most one row may span):
    greedy ids bit-exact and draws inside the nucleus; one token more is
    rejected with ValueError before any launch."""
    V, rows = 1 << 20, 2
    g = torch.Generator().manual_seed(34)
    logits = (torch.randn(rows, V, generator=g) * 2).to(torch.bfloat16)
    logits[0, V - 1] = 30.0  # the greedy row's max in the last chunk's last slot
    s = _sampler(dev, rows, seed=4)
    s.set_params([0.0, 0.8], [1.0, 0.5])
    got = s.sample(logits.to(dev)).cpu()
    assert int(got[0]) == V - 1 == int(osmp.greedy(logits)[0])
    probs = osmp.distribution(logits[1:], [0.8], [0.5])
    assert probs[0, got[1]] > 0
    with pytest.raises(ValueError, match="vocab"):
        s.sample(torch.zeros(rows, V + 1, dtype=torch.bfloat16, device=dev))


def test_largest_batch_twice(dev):
    """65,535 rows (the most one call takes; the last row's counter is the
    workspace's last), twice in a row on one workspace: greedy ids bit-exact,
    draws inside the nucleus; the second call starts from the counters the
    first left at zero."""
    rows, V = 65535, 200
    g = torch.Generator().manual_seed(35)
    s = _sampler(dev, rows, seed=5)
    temps = [0.0 if i % 3 == 0 else 0.8 for i in range(rows)]
    tops = [0.9 if i % 2 == 0 else 1.0 for i in range(rows)]
    s.set_params(temps, tops)
    greedy = torch.tensor([t == 0.0 for t in temps])
    sampled = ~greedy
    for call in range(2):
        logits = (torch.randn(rows, V, generator=g) * 2).to(torch.bfloat16)
        got = s.sample(logits.to(dev)).cpu()
        assert torch.equal(got[greedy], osmp.greedy(logits[greedy])), call
        # the oracle's nucleus is a per-row loop: every 97th sampled row and
        # the last rows (the highest counters) are checked
        idx = sampled.nonzero().flatten()
        idx = torch.cat([idx[::97], idx[-24:]])
        probs = osmp.distribution(logits[idx], [temps[i] for i in idx.tolist()], [tops[i] for i in idx.tolist()])
        kept = probs.gather(1, got[idx].view(-1, 1).long()).flatten()
        assert bool((kept > 0).all()), call


def test_reference_sample_semantics_on_the_gpu(dev):
    """The oracle's restatement of sample() (scheduler.py:310-316) against
    torch's own GPU kernels: a bf16 tensor divided by a Python float (the
    case where the reciprocal product and the quotient round apart, and every
    bf16 value in [1, 8) at 0.7), and F.softmax of bf16 logits without a
    dtype, whose bf16 probabilities lie within one bf16 step of the
    restatement's (the exponentials' last fp32 bits may differ)."""
    import torch.nn.functional as F

    x = torch.tensor([2.1765012589443917e-38]).to(torch.bfloat16)
    assert torch.equal((x.to(dev) / 0.3).cpu(), osmp.scalar_scaled_logits(x, 0.3))
    r = torch.arange(0x3F80, 0x4100, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    assert torch.equal((r.to(dev) / 0.7).cpu(), osmp.scalar_scaled_logits(r, 0.7))
    g = torch.Generator().manual_seed(2)
    logits = (torch.randn(32768, generator=g) * 3).to(torch.bfloat16)
    s = osmp.scalar_scaled_logits(logits, 0.7)
    got = F.softmax(s.to(dev), dim=-1).cpu()
    assert got.dtype == torch.bfloat16
    want = torch.softmax(s.float(), dim=-1).to(torch.bfloat16)
    steps = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs()
    assert int(steps.max()) <= 1
    p = osmp.sample_distribution(logits, 0.7)
    assert abs(float(p.sum()) - 1.0) < 1e-12 and torch.equal(p > 0, want > 0)
