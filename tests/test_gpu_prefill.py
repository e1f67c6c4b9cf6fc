"""GPU parity: ragged paged prefill attention (MFMA) vs the fp32 oracle.

Tolerance (the ``parity`` fixture): max-abs 2e-2 against the fp32 oracle on
bf16 inputs, and max |out - ref| / max(1, |ref|) <= 1.2e-2; each case's errors
are printed in the session's parity table.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as oatt
from tests.helpers import make_paged_batch

pytestmark = pytest.mark.gpu


def _run(dev, b, qo_lens, hq, hkv, d, causal=True, seed=0):
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    g = torch.Generator().manual_seed(seed)
    total = sum(qo_lens)
    q = torch.randn(total, hq, d, generator=g).to(torch.bfloat16)
    qo = [0]
    for x in qo_lens:
        qo.append(qo[-1] + x)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    w = BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    qo_d = torch.tensor(qo, dtype=torch.int32, device=dev)
    ip = torch.tensor(b["indptr"], dtype=torch.int32, device=dev)
    lp = torch.tensor(b["last"], dtype=torch.int32, device=dev)
    ix = b["indices"].to(dev)
    w.plan(qo_d, ip, ix, lp, hq, hkv, d, 16, causal=causal, pos_encoding_mode="NONE",
           q_data_type=torch.bfloat16)
    out = w.run(q.to(dev), b["pool"].to(dev))
    torch.cuda.synchronize()
    ref = oatt.prefill(q, b["pool"], qo, b["indptr"], b["indices"].tolist(), b["last"], causal=causal)
    return out.float().cpu(), ref


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128), (28, 4, 128), (64, 8, 128),
                                      (6, 3, 128), (8, 1, 64), (16, 4, 256), (8, 1, 256), (10, 2, 256),
                                      (40, 8, 128)])
@pytest.mark.parametrize("L", [1, 5, 64, 100, 300])
def test_single_request_causal(dev, parity, hq, hkv, d, L):
    b = make_paged_batch([L], hq, hkv, d, seed=L + d)
    out, ref = _run(dev, b, [L], hq, hkv, d, seed=L)
    parity(out, ref)


def test_ragged_batch(dev, parity):
    lens = [37, 200, 5, 513, 64, 1]
    b = make_paged_batch(lens, 32, 8, 128, seed=9)
    out, ref = _run(dev, b, lens, 32, 8, 128, seed=9)
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (14, 2, 64), (64, 8, 128), (16, 4, 256)])
def test_kv_longer_than_q_bottom_right_causal(dev, parity, hq, hkv, d):
    """Chunked-prefill shape: the last qo_len of kv_len tokens are queries
    (row blocks whose diagonal starts mid-tile, at every head_dim and group 8)."""
    kv_lens = [100, 260, 33]
    qo_lens = [20, 64, 33]
    b = make_paged_batch(kv_lens, hq, hkv, d, seed=4)
    out, ref = _run(dev, b, qo_lens, hq, hkv, d, seed=4)
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_zero_length_query_spans_in_a_ragged_batch(dev, parity, hq, hkv, d):
    """Requests with no query rows -- one with cached tokens, one empty --
    between requests with rows (one of them chunked: 10 rows over 64 tokens)
    get no tiles, and the rows around them are unaffected."""
    kv_lens = [37, 200, 0, 64, 1]
    qo_lens = [37, 0, 0, 10, 1]
    b = make_paged_batch(kv_lens, hq, hkv, d, seed=41)
    out, ref = _run(dev, b, qo_lens, hq, hkv, d, seed=41)
    assert out.shape[0] == sum(qo_lens)
    parity(out, ref)


@pytest.mark.parametrize("sm_scale", [0.3, 0.02])
def test_explicit_softmax_scale(dev, parity, sm_scale):
    """plan(sm_scale=...) replaces 1/sqrt(head_dim) in the causal prefill."""
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    hq, hkv, d = 32, 8, 128
    lens = [37, 300, 5]
    b = make_paged_batch(lens, hq, hkv, d, seed=58)
    g = torch.Generator().manual_seed(58)
    q = torch.randn(sum(lens), hq, d, generator=g).to(torch.bfloat16)
    qo = [0]
    for x in lens:
        qo.append(qo[-1] + x)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(torch.tensor(qo, dtype=torch.int32, device=dev), torch.tensor(b["indptr"], dtype=torch.int32, device=dev),
           b["indices"].to(dev), torch.tensor(b["last"], dtype=torch.int32, device=dev), hq, hkv, d, 16,
           causal=True, sm_scale=sm_scale)
    out = w.run(q.to(dev), b["pool"].to(dev)).float().cpu()
    ref = oatt.prefill(q, b["pool"], qo, b["indptr"], b["indices"].tolist(), b["last"], causal=True,
                       sm_scale=sm_scale)
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_large_scores_lazy_rescale(dev, parity, hq, hkv, d):
    """q and K scaled by 6: the row maxima grow past the lazy
    rescale margin many times along a row's key tiles."""
    lens = [300, 777]
    b = make_paged_batch(lens, hq, hkv, d, seed=62)
    b["pool"][:, 0] = (b["pool"][:, 0].float() * 6).to(torch.bfloat16)
    # V / 4 keeps the near one-hot outputs (single V entries) near unit size,
    # where the max-abs bound applies
    b["pool"][:, 1] = (b["pool"][:, 1].float() / 4).to(torch.bfloat16)
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    g = torch.Generator().manual_seed(62)
    q = (torch.randn(sum(lens), hq, d, generator=g) * 6).to(torch.bfloat16)
    qo = [0]
    for x in lens:
        qo.append(qo[-1] + x)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(torch.tensor(qo, dtype=torch.int32, device=dev), torch.tensor(b["indptr"], dtype=torch.int32, device=dev),
           b["indices"].to(dev), torch.tensor(b["last"], dtype=torch.int32, device=dev), hq, hkv, d, 16, causal=True)
    out = w.run(q.to(dev), b["pool"].to(dev)).float().cpu()
    assert torch.isfinite(out).all()
    ref = oatt.prefill(q, b["pool"], qo, b["indptr"], b["indices"].tolist(), b["last"], causal=True)
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (16, 4, 256)])
def test_head_major_q_and_out_views(dev, parity, hq, hkv, d):
    """q and out as head-major views ([heads, rows, head_dim] storage seen as
    [rows, heads, head_dim]: a head stride of rows * head_dim, larger than
    the row stride), as a single prompt's q.permute(0, 2, 1, 3).reshape(...)
    is when q is a contiguous [1, heads, seq, head_dim] tensor; every tile's
    rows and heads are read and written through them."""
    from minimal_inference_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    lens = [37, 300, 5, 129]
    b = make_paged_batch(lens, hq, hkv, d, seed=47)
    g = torch.Generator().manual_seed(47)
    q = torch.randn(sum(lens), hq, d, generator=g).to(torch.bfloat16)
    qo = [0]
    for x in lens:
        qo.append(qo[-1] + x)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=dev), "NHD")
    w.plan(torch.tensor(qo, dtype=torch.int32, device=dev), torch.tensor(b["indptr"], dtype=torch.int32, device=dev),
           b["indices"].to(dev), torch.tensor(b["last"], dtype=torch.int32, device=dev), hq, hkv, d, 16, causal=True)
    q_hm = q.transpose(0, 1).contiguous().to(dev).transpose(0, 1)
    out_hm = torch.full((hq, sum(lens), d), float("nan"), dtype=torch.bfloat16, device=dev).transpose(0, 1)
    assert q_hm.stride() == (d, sum(lens) * d, 1) and out_hm.stride() == q_hm.stride()
    got = w.run(q_hm, b["pool"].to(dev), out=out_hm)
    assert got.data_ptr() == out_hm.data_ptr()
    ref = oatt.prefill(q, b["pool"], qo, b["indptr"], b["indices"].tolist(), b["last"], causal=True)
    out = out_hm.float().cpu()
    assert torch.isfinite(out).all()
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(16, 4, 64), (32, 8, 128), (28, 4, 128), (16, 4, 256)])
def test_non_causal(dev, parity, hq, hkv, d):
    lens = [50, 129, 1, 300]
    b = make_paged_batch(lens, hq, hkv, d, seed=6)
    out, ref = _run(dev, b, lens, hq, hkv, d, causal=False, seed=6)
    parity(out, ref)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_non_causal_kv_longer_than_q(dev, parity, hq, hkv, d):
    """Non-causal rows over a longer cached context: every row sees every
    key, including the keys past its own position."""
    kv_lens = [100, 260, 33]
    qo_lens = [20, 64, 1]
    b = make_paged_batch(kv_lens, hq, hkv, d, seed=44)
    out, ref = _run(dev, b, qo_lens, hq, hkv, d, causal=False, seed=44)
    parity(out, ref)


def test_first_row_attends_only_to_token0(dev):
    """Causal row 0 sees one key, so its output is V[0] of its KV head."""
    b = make_paged_batch([40], 8, 2, 128, seed=12)
    out, _ = _run(dev, b, [40], 8, 2, 128, seed=12)
    page0 = int(b["indices"][0])
    v0 = b["pool"][page0, 1, 0].float().repeat_interleave(4, dim=0)
    assert torch.equal(out[0], v0)


def test_prefill_then_decode_consistency(dev, parity):
    """The last prefill row equals a decode query over the same context."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper

    lens = [77, 130]
    b = make_paged_batch(lens, 32, 8, 128, seed=15)
    out, _ = _run(dev, b, lens, 32, 8, 128, seed=15)
    g = torch.Generator().manual_seed(15)
    q = torch.randn(sum(lens), 32, 128, generator=g).to(torch.bfloat16)
    last_q = torch.stack([q[76], q[77 + 129]])
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    w = BatchDecodeWithPagedKVCacheWrapper(ws)
    w.plan(torch.tensor(b["indptr"], dtype=torch.int32, device=dev), b["indices"].to(dev),
           torch.tensor(b["last"], dtype=torch.int32, device=dev), 32, 8, 128, 16)
    dec = w.run(last_q.to(dev), b["pool"].to(dev)).float().cpu()
    parity(dec, torch.stack([out[76], out[77 + 129]]))


def _poison_tails(b):
    """NaN in every row past each request's length on its last page (K and V),
    where a pool holds stale data in practice; no result may read them."""
    pool = b["pool"].clone()
    idx = b["indices"].tolist()
    for r in range(len(b["last"])):
        lo, hi = b["indptr"][r], b["indptr"][r + 1]
        if hi > lo and b["last"][r] < 16:
            pool[idx[hi - 1], :, b["last"][r]:] = float("nan")
    return {**b, "pool": pool}


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64)])
def test_stale_rows_past_the_end_are_not_read(dev, parity, hq, hkv, d):
    lens = [37, 100, 5, 250]
    b = _poison_tails(make_paged_batch(lens, hq, hkv, d, seed=21))
    out, ref = _run(dev, b, lens, hq, hkv, d, seed=21)
    assert torch.isfinite(out).all()
    parity(out, ref)


def test_long_prompt_4096(dev, parity):
    """One 4,096-token causal prompt: 64 key tiles for the last query rows,
    the longest per-workgroup loop the bench batches do not reach."""
    b = make_paged_batch([4096], 8, 2, 128, seed=41)
    out, ref = _run(dev, b, [4096], 8, 2, 128, seed=41)
    parity(out, ref)
