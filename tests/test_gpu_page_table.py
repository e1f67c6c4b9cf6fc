"""GPU parity: device page table vs the oracle replay of the reference allocator.

indptr / indices / last_page_len of every decode step must be bit-exact with
the deque-based replay of scheduler.py's admission / growth / retirement
order; released pages must be zeroed in every layer and nothing else touched.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from oracle import paging as opg

pytestmark = pytest.mark.gpu


def _replay(dev, page_size, max_bs, max_seq, num_pages, requests, steps):
    """Drive DevicePageTable with the same trace as oracle.SchedulerTrace."""
    from minimal_inference_amd.kv_cache import DevicePageTable

    trace = opg.SchedulerTrace(max_bs, max_seq, page_size, max_num_pages=num_pages)
    for rid, (plen, mnt) in enumerate(requests):
        trace.submit(opg.TraceRequest(rid, plen, mnt))
    mpps = math.ceil(max_seq / page_size) + 1
    pt = DevicePageTable(num_pages, max_bs, mpps, page_size, dev)
    cap = max_bs * mpps + 64
    indptr = torch.zeros(max_bs + 1, dtype=torch.int32, device=dev)
    indices = torch.zeros(cap, dtype=torch.int32, device=dev)
    last = torch.zeros(max_bs, dtype=torch.int32, device=dev)
    bidx = torch.zeros(max_bs, dtype=torch.int32, device=dev)
    pos = torch.zeros(max_bs, dtype=torch.int32, device=dev)
    slot_of: dict[int, int] = {}
    free_slots = list(range(max_bs))
    checked = 0
    for _ in range(steps):
        res = trace.step()
        admits = []
        for rid, pages in res["admitted"]:
            slot_of[rid] = free_slots.pop(0)
            admits.append((slot_of[rid], len(pages)))
        dec = res["decode"]
        if admits and dec is None:
            # admission-only step: allocate with an empty CSR
            pt.step(admits, [], 0, indptr, indices, last, bidx, pos)
        if dec is not None:
            rows = [(slot_of[r], p) for r, p in zip(dec["rids"], dec["positions"])]
            pt.step(admits, rows, len(rows), indptr, indices, last, bidx, pos)
            n = len(rows)
            got_ptr = indptr[: n + 1].cpu().tolist()
            assert got_ptr == dec["indptr"]
            assert indices[: got_ptr[-1]].cpu().tolist() == dec["indices"]
            assert last[:n].cpu().tolist() == dec["last_page_len"]
            assert pos[:n].cpu().tolist() == dec["positions"]
            assert bidx[:n].cpu().tolist() == list(range(n))
            checked += 1
        for rid, _pages in res["released"]:
            pt.release(slot_of[rid])
            free_slots.append(slot_of.pop(rid))
        assert pt.free_count == len(trace.alloc.free_pages)
    assert pt.error_word() == 0
    return checked


def test_trace_matches_reference_allocator(dev):
    rnd = random.Random(3)
    reqs = [(rnd.randint(1, 200), rnd.randint(1, 60)) for _ in range(40)]
    checked = _replay(dev, 16, 8, 512, 200, reqs, 400)
    assert checked > 50


def test_trace_with_pool_pressure_and_wraparound(dev):
    """A small pool: admission stalls at the first request that does not fit
    and pages cycle through the ring many times.  Prompt + new tokens stay
    within 160 tokens (10 pages), and 6 slots x 10 pages fit in the 61 free
    pages, so decode growth -- which the reference does not gate on
    admission (scheduler.py:843-847) -- never exhausts the pool."""
    rnd = random.Random(11)
    reqs = [(rnd.randint(16, 120), rnd.randint(5, 40)) for _ in range(60)]
    checked = _replay(dev, 16, 6, 256, 62, reqs, 1500)
    assert checked > 100


def test_growth_exhaustion_raises_before_any_launch(dev):
    """Like allocate_pages (scheduler.py:210-213), growth beyond the pool raises."""
    from minimal_inference_amd.kv_cache import DevicePageTable

    pt = DevicePageTable(4, 2, 8, 16, dev)  # 3 allocatable pages
    buf = [torch.zeros(16, dtype=torch.int32, device=dev) for _ in range(5)]
    pt.step([(0, 2)], [], 0, *buf)
    pt.step([], [(0, 47)], 1, *buf)  # 48 tokens: grows to 3 pages, pool now empty
    with pytest.raises(RuntimeError):
        pt.step([], [(0, 48)], 1, *buf)  # 49 tokens would need a 4th page
    assert pt.free_count == 0
    assert pt.error_word() == 0


def test_graph_padding_rows_own_the_scratch_page(dev):
    from minimal_inference_amd.kv_cache import DevicePageTable

    pt = DevicePageTable(100, 4, 16, 16, dev)
    indptr = torch.zeros(9, dtype=torch.int32, device=dev)
    indices = torch.zeros(64, dtype=torch.int32, device=dev)
    last = torch.zeros(8, dtype=torch.int32, device=dev)
    bidx = torch.zeros(8, dtype=torch.int32, device=dev)
    pos = torch.zeros(8, dtype=torch.int32, device=dev)
    pt.step([(0, 2), (1, 1)], [(0, 20), (1, 3)], 8, indptr, indices, last, bidx, pos)
    ip = indptr.cpu().tolist()
    assert ip == [0, 2, 3, 4, 5, 6, 7, 8, 9]
    ix = indices[:9].cpu().tolist()
    assert ix[:3] == [0, 1, 2] and ix[3:] == [99] * 6
    assert last.cpu().tolist() == [5, 4, 1, 1, 1, 1, 1, 1]
    assert pos.cpu().tolist() == [20, 3, 0, 0, 0, 0, 0, 0]
    assert bidx.cpu().tolist() == list(range(8))


def test_release_zeroes_pages_in_every_layer(dev):
    from minimal_inference_amd.kv_cache import DevicePageTable, PagedKVCache

    kv = PagedKVCache(3, 2, 64, 4, 128, 16, dev, max_num_pages=20)
    kv.data.normal_()
    before = kv.data.clone()
    pt = DevicePageTable(20, 4, 8, 16, dev)
    ip = torch.zeros(5, dtype=torch.int32, device=dev)
    ix = torch.zeros(64, dtype=torch.int32, device=dev)
    z = torch.zeros(4, dtype=torch.int32, device=dev)
    pt.step([(0, 3), (1, 2)], [], 0, ip, ix, z, z.clone(), z.clone())
    pt.release(0)
    n = pt.step([], [], 0, ip, ix, z, z.clone(), z.clone())
    assert n == 3
    kv.zero_pages(pt.released, n)
    torch.cuda.synchronize()
    assert pt.released[:3].cpu().tolist() == [0, 1, 2]
    for p in range(20):
        if p in (0, 1, 2):
            assert int(kv.data[:, p].abs().sum()) == 0
        else:
            assert torch.equal(kv.data[:, p], before[:, p])
