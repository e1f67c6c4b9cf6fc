"""GPU parity: paged KV append vs the oracle (bit-exact, whole pool compared)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import paging as opg

pytestmark = pytest.mark.gpu


def _setup(lens, hkv, d, num_pages, seed):
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(num_pages, 2, 16, hkv, d, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_pages, generator=g)
    npages = [math.ceil(n / 16) for n in lens]
    indptr = [0]
    for n in npages:
        indptr.append(indptr[-1] + n)
    indices = perm[: indptr[-1]].to(torch.int32)
    last = [opg.last_page_len(n, 16) for n in lens]
    return g, pool, indptr, indices, last


def _run(dev, pool, k, v, bi, pos, indices, indptr, last):
    from minimal_inference_amd.page import append_paged_kv_cache

    pool_d = pool.to(dev)
    append_paged_kv_cache(
        k.to(dev) if k.device.type == "cpu" else k, v.to(dev) if v.device.type == "cpu" else v,
        torch.tensor(bi, dtype=torch.int32, device=dev), torch.tensor(pos, dtype=torch.int32, device=dev),
        pool_d, indices.to(dev), torch.tensor(indptr, dtype=torch.int32, device=dev),
        torch.tensor(last, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    return pool_d.cpu()


@pytest.mark.parametrize("hkv,d", [(2, 64), (8, 128), (4, 128), (8, 256)])
def test_decode_append_bit_exact(dev, hkv, d):
    lens = [17, 64, 203, 511, 1, 16]
    g, pool, indptr, indices, last = _setup(lens, hkv, d, 128, seed=hkv * 100 + d)
    k = torch.randn(len(lens), hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(len(lens), hkv, d, generator=g).to(torch.bfloat16)
    pos = [n - 1 for n in lens]
    bi = list(range(len(lens)))
    got = _run(dev, pool, k, v, bi, pos, indices, indptr, last)
    want = opg.append(pool, k, v, bi, pos, indices.tolist(), indptr)
    assert torch.equal(got, want)
    # the appended rows read back through the CSR gather
    for b, p in enumerate(pos):
        kk, vv = opg.gather_kv(got, indptr, indices.tolist(), last, b)
        assert torch.equal(kk[p], k[b]) and torch.equal(vv[p], v[b])


def test_prefill_append_strided_views(dev):
    """Prefill-shaped append from column slices of one fused qkv tensor."""
    hq, hkv, d = 14, 2, 64
    lens = [37, 200, 5]
    g, pool, indptr, indices, last = _setup(lens, hkv, d, 64, seed=7)
    total = sum(lens)
    qkv = torch.randn(total, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    qkv_d = qkv.to(dev)
    k_view = qkv_d[:, hq * d:(hq + hkv) * d].view(total, hkv, d)
    v_view = qkv_d[:, (hq + hkv) * d:].view(total, hkv, d)
    bi = [b for b, n in enumerate(lens) for _ in range(n)]
    pos = [i for n in lens for i in range(n)]
    got = _run(dev, pool, k_view, v_view, bi, pos, indices, indptr, last)
    want = opg.append(pool, qkv[:, hq * d:(hq + hkv) * d].view(total, hkv, d),
                      qkv[:, (hq + hkv) * d:].view(total, hkv, d), bi, pos, indices.tolist(), indptr)
    assert torch.equal(got, want)


def test_out_of_range_rows_not_written(dev):
    """Rows of requests without a page for their position write nothing."""
    hkv, d = 2, 64
    lens = [20, 0]
    g, pool, indptr, indices, last = _setup(lens, hkv, d, 16, seed=3)
    k = torch.randn(3, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(3, hkv, d, generator=g).to(torch.bfloat16)
    # request 0 owns 2 pages (positions 0..31); position 40 is outside; request 1 owns none
    bi, pos = [0, 0, 1], [19, 40, 0]
    got = _run(dev, pool, k, v, bi, pos, indices, indptr, last)
    want = opg.append(pool, k, v, bi, pos, indices.tolist(), indptr)
    assert torch.equal(got, want)
    changed = (got != pool).flatten(1).any(dim=1).nonzero().flatten().tolist()
    assert changed == [int(indices[1])]  # only page holding position 19


@pytest.mark.parametrize("hkv,d", [(2, 64), (8, 128)])
def test_unplaced_rows_among_placed_ones(dev, hkv, d):
    """A negative batch index, one past the batch, a negative position and a
    page id outside the pool write nothing, while the rows around them land;
    the K / V loads of every row are issued before its slot is known."""
    lens = [20, 40]
    g, pool, indptr, indices, last = _setup(lens, hkv, d, 16, seed=4)
    indices = indices.clone()
    indices[indptr[1] + 2] = pool.shape[0] + 5  # request 1's positions 32..39: a page outside the pool
    bi = [0, -1, 2, 1, 1, 1, 0]
    pos = [5, 3, 0, -3, 20, 35, 19]
    k = torch.randn(len(bi), hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(len(bi), hkv, d, generator=g).to(torch.bfloat16)
    got = _run(dev, pool, k, v, bi, pos, indices, indptr, last)
    ok = [i for i in range(len(bi)) if 0 <= bi[i] < len(lens) and pos[i] >= 0]
    want = opg.append(pool, k[ok], v[ok], [bi[i] for i in ok], [pos[i] for i in ok], indices.tolist(), indptr)
    assert torch.equal(got, want)
    changed = set((got != pool).flatten(1).any(dim=1).nonzero().flatten().tolist())
    # request 0's positions 5 and 19 (its pages 0 and 1), request 1's position 20 (its page 1)
    assert changed == {int(indices[0]), int(indices[1]), int(indices[indptr[1] + 1])}


def test_empty_append_is_noop(dev):
    from minimal_inference_amd.page import append_paged_kv_cache

    pool = torch.zeros(4, 2, 16, 2, 64, dtype=torch.bfloat16, device=dev)
    e = torch.empty(0, 2, 64, dtype=torch.bfloat16, device=dev)
    z = torch.zeros(0, dtype=torch.int32, device=dev)
    ip = torch.zeros(1, dtype=torch.int32, device=dev)
    append_paged_kv_cache(e, e, z, z, pool, z, ip, z)
    torch.cuda.synchronize()
    assert int(pool.abs().sum()) == 0


def test_rejects_bad_arguments(dev):
    from minimal_inference_amd.page import append_paged_kv_cache

    pool = torch.zeros(4, 2, 16, 2, 64, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, 2, 64, dtype=torch.bfloat16, device=dev)
    one = torch.zeros(1, dtype=torch.int32, device=dev)
    ip = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        append_paged_kv_cache(k.float(), k, one, one, pool, one, ip, one)
    with pytest.raises(ValueError):
        append_paged_kv_cache(k, k, one.long(), one, pool, one, ip, one)
    with pytest.raises(ValueError):
        append_paged_kv_cache(k, k, one, one, pool, one, ip, one, kv_layout="HND")
