"""GPU parity: fused RoPE + paged KV append vs the oracle's unfused sequence.

Bar: bit-exact for the rotated q and for the whole pool (rotated k, v in
their slots, every other slot unchanged) -- the kernel evaluates the same
bf16 roundings as the reference's RoPE ops (model.py:92-107).
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import paging as opg
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def _case(lens, new_pos, hq, hkv, d, num_pages, seed, extra_cols=0):
    """One request per entry of ``lens`` (pages for its length), tokens at
    ``new_pos`` [(request, position)]; qkv rows with ``extra_cols`` of slack."""
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(num_pages, 2, 16, hkv, d, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_pages, generator=g)
    npages = [math.ceil(n / 16) for n in lens]
    indptr = [0]
    for n in npages:
        indptr.append(indptr[-1] + n)
    indices = perm[: indptr[-1]].to(torch.int32)
    last = [opg.last_page_len(n, 16) for n in lens]
    width = (hq + 2 * hkv) * d
    qkv_full = (torch.randn(len(new_pos), width + extra_cols, generator=g) * 3).to(torch.bfloat16)
    return pool, indptr, indices, last, qkv_full


def _run(dev, qkv_full, width, hq, hkv, rope_pos, cos, sin, bi, pos, pool, indices, indptr, last, separate_q):
    from minimal_inference_amd.page import rope_append_paged_kv_cache

    qkv_d = qkv_full.to(dev)[:, :width]
    pool_d = pool.to(dev)
    d = pool.shape[-1]
    q_out = torch.full((qkv_full.shape[0], hq, d), 7.0, dtype=torch.bfloat16, device=dev) if separate_q else None
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    q = rope_append_paged_kv_cache(qkv_d, hq, hkv, i32(rope_pos), cos.to(dev), sin.to(dev), i32(bi), i32(pos),
                                   pool_d, indices.to(dev), i32(indptr), i32(last), q_out=q_out)
    torch.cuda.synchronize()
    return q.cpu(), pool_d.cpu(), qkv_d.cpu()


@pytest.mark.parametrize("hq,hkv,d,theta", [(32, 8, 128, 1e6), (14, 2, 64, 1e6), (28, 4, 128, 1e6),
                                            (64, 8, 128, 1e6), (8, 8, 256, 1e4), (12, 4, 64, 1e4)])
@pytest.mark.parametrize("separate_q", [False, True])
def test_decode_rows_bit_exact(dev, hq, hkv, d, theta, separate_q):
    lens = [17, 64, 203, 511, 1, 16, 900]
    pool, indptr, indices, last, qkv = _case(lens, [(b, n - 1) for b, n in enumerate(lens)], hq, hkv, d, 160,
                                             seed=hq * 31 + d)
    cos, sin = orope.tables(d, 1024, theta)
    pos = [n - 1 for n in lens]
    bi = list(range(len(lens)))
    width = (hq + 2 * hkv) * d
    q, got_pool, _ = _run(dev, qkv, width, hq, hkv, pos, cos, sin, bi, pos, pool, indices, indptr, last, separate_q)
    want_q, want_pool = orope.rope_append(qkv[:, :width], hq, hkv, pos, cos, sin, pool, indptr, indices.tolist(),
                                          bi, pos)
    assert torch.equal(q, want_q)
    assert torch.equal(got_pool, want_pool)


def test_prefill_rows_strided_and_in_place(dev):
    """Prefill-shaped: every position of three prompts, qkv rows with slack
    columns (row stride > (Hq + 2 Hkv) * D); q is rotated in place and the
    slack and v columns of qkv are untouched."""
    hq, hkv, d = 14, 2, 64
    lens = [5, 33, 48]
    toks = [(b, p) for b, n in enumerate(lens) for p in range(n)]
    pool, indptr, indices, last, qkv = _case(lens, toks, hq, hkv, d, 40, seed=9, extra_cols=64)
    cos, sin = orope.tables(d, 64, 1e6)
    bi = [b for b, _ in toks]
    pos = [p for _, p in toks]
    width = (hq + 2 * hkv) * d
    q, got_pool, qkv_after = _run(dev, qkv, width, hq, hkv, pos, cos, sin, bi, pos, pool, indices, indptr, last,
                                  separate_q=False)
    want_q, want_pool = orope.rope_append(qkv[:, :width], hq, hkv, pos, cos, sin, pool, indptr, indices.tolist(),
                                          bi, pos)
    assert torch.equal(q, want_q)
    assert torch.equal(got_pool, want_pool)
    assert torch.equal(qkv_after[:, hq * d:width], qkv[:, hq * d:width])  # k, v columns read only
    assert torch.equal(qkv_after[:, : hq * d].view(-1, hq, d), want_q)


def test_rows_outside_page_list_and_clamped_positions(dev):
    """Rows whose slot is outside the request's pages are not appended (q is
    still rotated); rope positions beyond the table use its last row."""
    hq, hkv, d = 8, 2, 64
    lens = [16, 20]
    pool, indptr, indices, last, qkv = _case(lens, [(0, 0)] * 4, hq, hkv, d, 12, seed=5)
    cos, sin = orope.tables(d, 32, 1e4)
    bi = [0, 0, 1, 1]
    pos = [3, 16, 19, 40]           # (0, 16) and (1, 40) fall outside the page lists
    rope_pos = [3, 100, 19, 40]     # 100 and 40 clamp to row 31
    width = (hq + 2 * hkv) * d
    q, got_pool, _ = _run(dev, qkv, width, hq, hkv, rope_pos, cos, sin, bi, pos, pool, indices, indptr, last,
                          separate_q=True)
    want_q, want_pool = orope.rope_append(qkv[:, :width], hq, hkv, rope_pos, cos, sin, pool, indptr,
                                          indices.tolist(), bi, pos)
    assert torch.equal(q, want_q)
    assert torch.equal(got_pool, want_pool)


def test_model_forward_fused_equals_unfused(dev):
    """End to end: greedy trajectories of the fused and unfused model are identical."""
    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    cfg = PRESETS["qwen2.5-0.5b"]
    outs = []
    for fused in (True, False):
        model = Model(cfg, dev, seed=3, max_positions=512, fused_rope=fused)
        sch = Scheduler(model, max_batch_size=4, max_seq_len=256, seed=3, use_graphs=False)
        g = torch.Generator().manual_seed(8)
        reqs = [Request(str(i), torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist(), 6, 0.0, 1.0)
                for i, n in enumerate([9, 40, 77])]
        for r in reqs:
            sch.submit(r)
        while any(r.status.value != "finished" for r in reqs):
            sch.step()
        outs.append([r.generated_tokens for r in reqs])
    assert outs[0] == outs[1]


@pytest.mark.parametrize("hq,hkv,d,theta", [(32, 8, 128, 1e6), (14, 2, 64, 1e6), (28, 4, 128, 1e6),
                                            (64, 8, 128, 1e6), (8, 8, 256, 1e4), (12, 4, 64, 1e4),
                                            (6, 3, 128, 1e4)])
def test_decode_attention_with_rope_append_equals_the_three_calls(dev, parity, hq, hkv, d, theta):
    """run_rope_append (RoPE of q and k, the K/V append and decode attention
    in one launch) against rope_append_paged_kv_cache followed by the
    wrapper's run on the rotated q: bit-identical output and pool, qkv left
    unmodified; requests from 1 token (the new one alone) to 5,000 (many
    splits, page groups past the inline ids), new tokens on the first and
    last row of a page; the output within the oracle's bound."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    from minimal_inference_amd.page import rope_append_paged_kv_cache
    from oracle import attention as oatt

    lens = [1, 2, 16, 17, 64, 203, 511, 900, 1024, 2049, 5000, 33]
    pages = sum(math.ceil(n / 16) for n in lens) + 8
    pool, indptr, indices, last, qkv = _case(lens, [(b, n - 1) for b, n in enumerate(lens)], hq, hkv, d, pages,
                                             seed=hq * 13 + d)
    qkv = (qkv.float() / 3).to(torch.bfloat16)  # N(0, 1) rows, the scale of the other decode parity cases
    cos, sin = orope.tables(d, 8192, theta)
    pos = [n - 1 for n in lens]
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    cos_d, sin_d, ip, ix, lp = cos.to(dev), sin.to(dev), i32(indptr), indices.to(dev), i32(last)
    outs, pools = [], []
    for fused in (False, True):
        w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev))
        w.plan(ip, ix, lp, hq, hkv, d, 16)
        pool_d = pool.to(dev)
        qkv_d = qkv.to(dev)
        if fused:
            o = w.run_rope_append(qkv_d, cos_d, sin_d, pool_d)
            torch.cuda.synchronize()
            assert torch.equal(qkv_d.cpu(), qkv)
        else:
            q = rope_append_paged_kv_cache(qkv_d, hq, hkv, i32(pos), cos_d, sin_d, i32(list(range(len(lens)))),
                                           i32(pos), pool_d, ix, ip, lp)
            o = w.run(q, pool_d)
        torch.cuda.synchronize()
        outs.append(o.cpu())
        pools.append(pool_d.cpu())
    assert torch.equal(pools[1], pools[0])
    assert torch.equal(outs[1], outs[0])
    want_q, want_pool = orope.rope_append(qkv, hq, hkv, pos, cos, sin, pool, indptr, indices.tolist(),
                                          list(range(len(lens))), pos)
    assert torch.equal(pools[1], want_pool)
    parity(outs[1].float(), oatt.decode(want_q, want_pool, indptr, indices.tolist(), last))


def test_engine_decode_with_and_without_the_fused_launch(dev):
    """The engine (graphs, 8 slots, padded batches) with the decode step's
    RoPE + append inside the attention launch and with the separate launch:
    identical greedy tokens step for step."""
    from minimal_inference_amd.engine import Request, Scheduler
    from minimal_inference_amd.model import PRESETS, Model

    cfg = PRESETS["qwen2.5-0.5b"]
    cfg = type(cfg)(**{**cfg.__dict__, "num_hidden_layers": 6})
    outs = []
    for fused_decode in (True, False):
        model = Model(cfg, dev, seed=4, max_positions=1024, fused_decode=fused_decode)
        sch = Scheduler(model, max_batch_size=8, max_seq_len=512, seed=4)
        g = torch.Generator().manual_seed(9)
        reqs = [Request(str(i), torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist(), 20, 0.0, 1.0)
                for i, n in enumerate([9, 40, 77, 16, 1, 130])]
        for r in reqs:
            sch.submit(r)
        while sch.has_work():
            sch.step()
        assert sch.pt.error_word() == 0
        outs.append([r.generated_tokens for r in reqs])
    assert outs[0] == outs[1]
