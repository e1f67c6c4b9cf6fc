"""The reference's own call forms, keyword for keyword, against the oracle.

One prefill and one decode step of one layer, written the way the reference
writes them:
- the wrappers are built as at scheduler.py:528-539 (a uint8 workspace,
  kv_layout="NHD");
- they are planned with scheduler.py:704-716's and 905-916's keywords;
- K / V are appended with model.py:207-216's positional call, from
  [bsz, kv_heads, seq, head_dim] tensors reshaped as model.py:203-204 does;
- the wrappers run on Q padded per KV group to a power-of-two group
  (model.py:218-230, 14 -> 16 heads for Qwen2.5-0.5B), and the padded heads
  are stripped afterwards (model.py:236-240).

Tolerance: the ``parity`` fixture (max-abs 2e-2 against the fp32 oracle);
pools bit-exact against the oracle's append.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import paging as opg
from tests.helpers import make_paged_batch

pytestmark = pytest.mark.gpu


def _padded_group(group: int) -> int:
    return 1 << (group - 1).bit_length()


def _pad_heads(q_fi: torch.Tensor, hkv: int, group: int) -> torch.Tensor:
    leading = q_fi.shape[:-2]
    pg = _padded_group(group)
    q_fi = q_fi.view(*leading, hkv, group, q_fi.shape[-1])
    q_fi = F.pad(q_fi, (0, 0, 0, pg - group))
    return q_fi.reshape(*leading, hkv * pg, q_fi.shape[-1])


def _strip_heads(out: torch.Tensor, hkv: int, group: int) -> torch.Tensor:
    leading = out.shape[:-2]
    pg = _padded_group(group)
    return out.view(*leading, hkv, pg, out.shape[-1])[..., :group, :].reshape(*leading, hkv * group, out.shape[-1])


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128), (28, 4, 128)])
def test_prefill_step_in_the_reference_call_form(dev, parity, hq, hkv, d):
    from minimal_inference_amd.page import append_paged_kv_cache
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    L = 77
    g = torch.Generator().manual_seed(hq + d)
    pages = 5  # 80 slots for 77 tokens
    pool = torch.randn(12, 2, 16, hkv, d, generator=g).to(torch.bfloat16)
    page_list = torch.randperm(12, generator=g)[:pages].to(torch.int32)
    q = torch.randn(1, hq, L, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, hkv, L, d, generator=g).to(torch.bfloat16)
    v = torch.randn(1, hkv, L, d, generator=g).to(torch.bfloat16)

    kv_data = pool.to(dev)
    qo_indptr = torch.tensor([0, L], dtype=torch.int32, device=dev)
    kv_page_indptr = torch.tensor([0, pages], dtype=torch.int32, device=dev)
    kv_page_indices = page_list.to(dev)
    kv_last_page_len = torch.tensor([opg.last_page_len(L, 16)], dtype=torch.int32, device=dev)
    batch_indices = torch.zeros(L, dtype=torch.int32, device=dev)
    positions = torch.arange(L, dtype=torch.int32, device=dev)

    group = hq // hkv
    padded = hkv * _padded_group(group)
    wrapper = BatchPrefillWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev),
                                                  kv_layout="NHD")
    wrapper.plan(
        qo_indptr=qo_indptr,
        paged_kv_indptr=kv_page_indptr,
        paged_kv_indices=kv_page_indices,
        paged_kv_last_page_len=kv_last_page_len,
        num_qo_heads=padded,
        num_kv_heads=hkv,
        head_dim_qk=d,
        page_size=16,
        causal=True,
        pos_encoding_mode="NONE",
        q_data_type=torch.bfloat16,
    )
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    k_append = kd.permute(0, 2, 1, 3).reshape(-1, hkv, d)
    v_append = vd.permute(0, 2, 1, 3).reshape(-1, hkv, d)
    append_paged_kv_cache(k_append, v_append, batch_indices, positions, kv_data, kv_page_indices,
                          kv_page_indptr, kv_last_page_len)
    q_fi = qd.permute(0, 2, 1, 3).reshape(-1, hq, d)
    if padded != hq:
        q_fi = _pad_heads(q_fi, hkv, group)
    out = wrapper.run(q_fi, kv_data)
    if padded != hq:
        out = _strip_heads(out, hkv, group)
    torch.cuda.synchronize()

    k_rows = k.permute(0, 2, 1, 3).reshape(-1, hkv, d)
    v_rows = v.permute(0, 2, 1, 3).reshape(-1, hkv, d)
    want_pool = opg.append(pool, k_rows, v_rows, [0] * L, list(range(L)), page_list.tolist(), [0, pages])
    assert torch.equal(kv_data.cpu(), want_pool)
    ref = oatt.prefill(q.permute(0, 2, 1, 3).reshape(-1, hq, d), want_pool, [0, L], [0, pages], page_list.tolist(),
                       [opg.last_page_len(L, 16)], causal=True)
    assert out.shape == (L, hq, d)
    parity(out.float().cpu(), ref)


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128), (28, 4, 128)])
def test_decode_step_in_the_reference_call_form(dev, parity, hq, hkv, d):
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    from minimal_inference_amd.page import append_paged_kv_cache

    lens = [17, 64, 203, 511, 1, 16]  # tokens after this step's append
    B = len(lens)
    b = make_paged_batch(lens, hq, hkv, d, seed=hq * 3 + d)
    g = torch.Generator().manual_seed(d)
    q = torch.randn(B, hq, 1, d, generator=g).to(torch.bfloat16)
    k = torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16)

    kv_data = b["pool"].to(dev)
    kv_page_indptr = torch.tensor(b["indptr"], dtype=torch.int32, device=dev)
    kv_page_indices = b["indices"].to(dev)
    kv_last_page_len = torch.tensor(b["last"], dtype=torch.int32, device=dev)
    batch_indices = torch.arange(B, dtype=torch.int32, device=dev)
    positions = torch.tensor([n - 1 for n in lens], dtype=torch.int32, device=dev)

    group = hq // hkv
    padded = hkv * _padded_group(group)
    wrapper = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev),
                                                 kv_layout="NHD")
    wrapper.plan(
        indptr=kv_page_indptr,
        indices=kv_page_indices,
        last_page_len=kv_last_page_len,
        num_qo_heads=padded,
        num_kv_heads=hkv,
        head_dim=d,
        page_size=16,
        pos_encoding_mode="NONE",
        q_data_type=torch.bfloat16,
        data_type=torch.bfloat16,
    )
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    k_append = kd.permute(0, 2, 1, 3).reshape(-1, hkv, d)
    v_append = vd.permute(0, 2, 1, 3).reshape(-1, hkv, d)
    append_paged_kv_cache(k_append, v_append, batch_indices, positions, kv_data, kv_page_indices,
                          kv_page_indptr, kv_last_page_len)
    q_fi = qd.squeeze(2)
    if padded != hq:
        q_fi = _pad_heads(q_fi, hkv, group)
    out = wrapper.run(q_fi, kv_data)
    if padded != hq:
        out = _strip_heads(out, hkv, group)
    torch.cuda.synchronize()

    want_pool = opg.append(b["pool"], k[:, :, 0], v[:, :, 0], list(range(B)), [n - 1 for n in lens],
                           b["indices"].tolist(), b["indptr"])
    assert torch.equal(kv_data.cpu(), want_pool)
    ref = oatt.decode(q[:, :, 0], want_pool, b["indptr"], b["indices"].tolist(), b["last"])
    assert out.shape == (B, hq, d)
    parity(out.float().cpu(), ref)


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128)])
def test_decode_graph_runner_in_the_reference_call_form(dev, parity, hq, hkv, d):
    """The reference's graph runner (scheduler.py:353-469, 900-916): static
    buffers initialised as at scheduler.py:366-374 (indptr zeros, indices all
    the scratch page, last_page_len ones, batch_indices arange, positions
    zeros); a plan on that dummy metadata with indices sliced to the batch
    size (scheduler.py:402-413); three warm-up passes of append + run on a
    side stream and one captured pass; then, per step, the real metadata
    copied into the static buffers, a plan on slices of them outside the
    graph, and a replay. Pools bit-exact and outputs within the parity bar
    at every replay."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    from minimal_inference_amd.page import append_paged_kv_cache

    B, num_pages, max_num_pages = 8, 400, 512
    scratch_page = num_pages - 1
    group = hq // hkv
    padded = hkv * _padded_group(group)
    kv_page_indptr = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    kv_page_indices = torch.full((max_num_pages,), scratch_page, dtype=torch.int32, device=dev)
    kv_last_page_len = torch.ones(B, dtype=torch.int32, device=dev)
    batch_indices = torch.arange(B, dtype=torch.int32, device=dev)
    positions = torch.zeros(B, dtype=torch.int32, device=dev)
    q_in = torch.zeros(B, hq, 1, d, dtype=torch.bfloat16, device=dev)
    k_in = torch.zeros(B, hkv, 1, d, dtype=torch.bfloat16, device=dev)
    v_in = torch.zeros(B, hkv, 1, d, dtype=torch.bfloat16, device=dev)
    kv_data = torch.zeros(num_pages, 2, 16, hkv, d, dtype=torch.bfloat16, device=dev)

    wrapper = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=dev),
                                                 kv_layout="NHD")
    plan_kw = dict(num_qo_heads=padded, num_kv_heads=hkv, head_dim=d, page_size=16, pos_encoding_mode="NONE",
                   q_data_type=torch.bfloat16, data_type=torch.bfloat16)
    wrapper.plan(indptr=kv_page_indptr, indices=kv_page_indices[:B], last_page_len=kv_last_page_len, **plan_kw)

    def layer():
        k_append = k_in.permute(0, 2, 1, 3).reshape(-1, hkv, d)
        v_append = v_in.permute(0, 2, 1, 3).reshape(-1, hkv, d)
        append_paged_kv_cache(k_append, v_append, batch_indices, positions, kv_data, kv_page_indices,
                              kv_page_indptr, kv_last_page_len)
        q_fi = q_in.squeeze(2)
        if padded != hq:
            q_fi = _pad_heads(q_fi, hkv, group)
        out = wrapper.run(q_fi, kv_data)
        return _strip_heads(out, hkv, group) if padded != hq else out

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            layer()
    s.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer()

    g = torch.Generator().manual_seed(d + hq)
    for step, lens in enumerate([[40, 1, 300, 17, 64, 129, 5, 16], [41, 2, 301, 18, 65, 130, 6, 17],
                                 [900, 33, 2, 1, 1000, 16, 17, 250]]):
        b = make_paged_batch(lens, hq, hkv, d, num_pages=num_pages - 1, seed=step + 70)
        pool = torch.cat([b["pool"], torch.zeros(1, 2, 16, hkv, d, dtype=torch.bfloat16)])
        kv_data.copy_(pool)
        q = torch.randn(B, hq, 1, d, generator=g).to(torch.bfloat16)
        k = torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16)
        v = torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16)
        q_in.copy_(q)
        k_in.copy_(k)
        v_in.copy_(v)
        n_idx = b["indices"].numel()
        kv_page_indptr.copy_(torch.tensor(b["indptr"], dtype=torch.int32))
        kv_page_indices[:n_idx].copy_(b["indices"])
        kv_last_page_len.copy_(torch.tensor(b["last"], dtype=torch.int32))
        positions.copy_(torch.tensor([n - 1 for n in lens], dtype=torch.int32))
        wrapper.plan(indptr=kv_page_indptr[:B + 1], indices=kv_page_indices[:n_idx],
                     last_page_len=kv_last_page_len[:B], **plan_kw)
        graph.replay()
        torch.cuda.synchronize()
        want_pool = opg.append(pool, k[:, :, 0], v[:, :, 0], list(range(B)), [n - 1 for n in lens],
                               b["indices"].tolist(), b["indptr"])
        assert torch.equal(kv_data.cpu(), want_pool), step
        ref = oatt.decode(q[:, :, 0], want_pool, b["indptr"], b["indices"].tolist(), b["last"])
        parity(out.float().cpu(), ref, f"step {step}")
