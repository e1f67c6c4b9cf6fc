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
