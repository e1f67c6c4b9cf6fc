"""CPU: pin the attention oracle.

Against (a) a float64 brute force written as explicit per-token loops with
math.exp (a different formulation from the oracle's batched matmul/softmax),
(b) torch's scaled_dot_product_attention on the gathered tensors, and
(c) closed forms: kv_len 1 -> V[0]; identical keys -> mean of V; one dominant
logit -> that V row; causal row 0 -> V[0].  A dropped scale, a transposed
GQA mapping (h % hkv instead of h // group) or a mask off by one fails these.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import paging as opg
from tests.helpers import make_paged_batch


def brute_decode(q, pool, indptr, indices, last):
    b_count, hq, d = q.shape
    hkv = pool.shape[3]
    group = hq // hkv
    out = torch.zeros(b_count, hq, d, dtype=torch.float64)
    for b in range(b_count):
        k, v = opg.gather_kv(pool, indptr, indices, last, b)
        for h in range(hq):
            kh = h // group
            logits = [sum(float(q[b, h, i]) * float(k[t, kh, i]) for i in range(d)) / math.sqrt(d)
                      for t in range(k.shape[0])]
            if not logits:
                continue
            m = max(logits)
            w = [math.exp(x - m) for x in logits]
            z = sum(w)
            for i in range(d):
                out[b, h, i] = sum(w[t] * float(v[t, kh, i]) for t in range(k.shape[0])) / z
    return out


def test_decode_vs_float64_brute_force():
    b = make_paged_batch([1, 7, 17, 33], 6, 2, 8, seed=1)
    got = oatt.decode(b["q"], b["pool"], b["indptr"], b["indices"].tolist(), b["last"])
    want = brute_decode(b["q"], b["pool"], b["indptr"], b["indices"].tolist(), b["last"])
    assert (got.double() - want).abs().max().item() < 1e-5


def test_decode_vs_sdpa():
    b = make_paged_batch([17, 64, 203, 511], 14, 2, 64, num_pages=128, seed=0)
    got = oatt.decode(b["q"], b["pool"], b["indptr"], b["indices"].tolist(), b["last"])
    for r in range(4):
        k, v = opg.gather_kv(b["pool"], b["indptr"], b["indices"].tolist(), b["last"], r)
        qf = b["q"][r].float().unsqueeze(1)  # [H, 1, D]
        kf = k.float().transpose(0, 1).repeat_interleave(7, dim=0)
        vf = v.float().transpose(0, 1).repeat_interleave(7, dim=0)
        ref = F.scaled_dot_product_attention(qf, kf, vf)[:, 0]
        assert (got[r] - ref).abs().max().item() < 1e-5


def test_decode_closed_forms():
    b = make_paged_batch([1, 40, 40], 4, 2, 16, seed=3)
    pool = b["pool"].clone()
    ix = b["indices"].tolist()
    # request 1: identical keys -> uniform weights
    for p in ix[b["indptr"][1]:b["indptr"][2]]:
        pool[p, 0] = pool[ix[b["indptr"][1]], 0, 0]
    # request 2: key 9 aligned with q scaled up -> dominant
    q = b["q"].clone()
    k2, _ = opg.gather_kv(pool, b["indptr"], ix, b["last"], 2)
    page, slot = ix[b["indptr"][2] + 9 // 16], 9 % 16
    pool[page, 0, slot] = (q[2, ::2] * 64).to(torch.bfloat16)  # heads 0, 2 -> kv heads 0, 1
    got = oatt.decode(q, pool, b["indptr"], ix, b["last"])
    _, v0 = opg.gather_kv(pool, b["indptr"], ix, b["last"], 0)
    assert torch.allclose(got[0], v0[0].float().repeat_interleave(2, dim=0))
    _, v1 = opg.gather_kv(pool, b["indptr"], ix, b["last"], 1)
    assert torch.allclose(got[1], v1.float().mean(0).repeat_interleave(2, dim=0), atol=1e-5)
    _, v2 = opg.gather_kv(pool, b["indptr"], ix, b["last"], 2)
    assert torch.allclose(got[2, 0], v2[9, 0].float(), atol=1e-3)
    assert torch.allclose(got[2, 2], v2[9, 1].float(), atol=1e-3)


def test_gqa_head_mapping_is_h_div_group():
    """Q head h reads KV head h // group (repeat_interleave, model.py:287-288)."""
    b = make_paged_batch([5], 8, 2, 16, seed=8)
    pool = b["pool"].clone()
    pool[:, 1, :, 1] = 0  # zero V of kv head 1
    got = oatt.decode(b["q"], pool, b["indptr"], b["indices"].tolist(), b["last"])
    assert got[0, 4:].abs().max() == 0 and got[0, :4].abs().max() > 0


def test_prefill_causal_vs_sdpa_and_row0():
    b = make_paged_batch([50], 4, 2, 16, seed=5)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(50, 4, 16, generator=g).to(torch.bfloat16)
    got = oatt.prefill(q, b["pool"], [0, 50], b["indptr"], b["indices"].tolist(), b["last"], causal=True)
    k, v = opg.gather_kv(b["pool"], b["indptr"], b["indices"].tolist(), b["last"], 0)
    ref = F.scaled_dot_product_attention(q.float().transpose(0, 1),
                                         k.float().transpose(0, 1).repeat_interleave(2, 0),
                                         v.float().transpose(0, 1).repeat_interleave(2, 0), is_causal=True)
    assert (got - ref.transpose(0, 1)).abs().max().item() < 1e-5
    assert torch.allclose(got[0], v[0].float().repeat_interleave(2, dim=0))


def test_prefill_bottom_right_alignment():
    """kv_len > qo_len: the last query row sees every key (mask offset kv-qo)."""
    b = make_paged_batch([40], 2, 1, 8, seed=6)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(10, 2, 8, generator=g).to(torch.bfloat16)
    got = oatt.prefill(q, b["pool"], [0, 10], b["indptr"], b["indices"].tolist(), b["last"], causal=True)
    full = oatt.decode(q[9:10], b["pool"], b["indptr"], b["indices"].tolist(), b["last"])
    assert torch.allclose(got[9], full[0], atol=1e-6)
    k, v = opg.gather_kv(b["pool"], b["indptr"], b["indices"].tolist(), b["last"], 0)
    sub = opg.build_csr([b["indices"].tolist()[:2]], [31], 16)
    first = oatt.decode(q[0:1], b["pool"], sub[0], sub[1], sub[2])
    assert torch.allclose(got[0], first[0], atol=1e-6)  # row 0 sees keys 0..30
