"""CPU: pin the paging oracle (allocator replay, CSR, padding, append).

Checks are closed forms and invariants that a plausible slip (LIFO instead of
FIFO, off-by-one in last_page_len, wrong page index for a position) fails.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from oracle import paging as opg


def test_fifo_order_hand_trace():
    a = opg.ReferenceAllocator(8)  # pages 0..6 free, 7 is scratch
    assert a.scratch_page == 7
    assert a.allocate_pages(3) == [0, 1, 2]
    assert a.allocate_pages(2) == [3, 4]
    a.release_pages([1, 0, 2])
    # FIFO: the never-used pages come first, then released pages in release order
    assert a.allocate_pages(4) == [5, 6, 1, 0]
    assert a.allocate_pages(1) == [2]
    with pytest.raises(RuntimeError):
        a.allocate_pages(1)


def test_for_config_page_count():
    # scheduler.py:191-192: max_bs * ceil(max_seq / page_size)
    assert opg.ReferenceAllocator.for_config(40, 4096, 16).max_num_pages == 40 * 256
    assert opg.ReferenceAllocator.for_config(3, 100, 16).max_num_pages == 3 * 7


@pytest.mark.parametrize("n", list(range(0, 70)))
def test_last_page_len_reconstructs_length(n):
    ps = 16
    npages = math.ceil(n / ps)
    last = opg.last_page_len(n, ps)
    if n == 0:
        assert last == 0 and npages == 0
    else:
        assert 1 <= last <= ps
        assert (npages - 1) * ps + last == n


def test_build_csr_concatenates_in_request_order():
    ip, ix, last = opg.build_csr([[5, 6], [], [9, 1, 3]], [20, 0, 33], 16)
    assert ip == [0, 2, 2, 5]
    assert ix == [5, 6, 9, 1, 3]
    assert last == [4, 0, 1]


def test_decode_padding_rows_use_scratch():
    ip, ix, last, bi, pos = opg.decode_padding([0, 2], [4, 5], [3], [18], 4, 99)
    assert ip == [0, 2, 3, 4, 5] and ix == [4, 5, 99, 99, 99]
    assert last == [3, 1, 1, 1] and pos == [18, 0, 0, 0] and bi == [0, 1, 2, 3]


def test_append_round_trip_and_untouched_slots():
    g = torch.Generator().manual_seed(0)
    pool = torch.randn(10, 2, 16, 2, 8, generator=g).to(torch.bfloat16)
    ip, ix, last = opg.build_csr([[7, 2], [4]], [20, 5], 16)
    k = torch.randn(3, 2, 8, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 2, 8, generator=g).to(torch.bfloat16)
    out = opg.append(pool, k, v, [0, 0, 1], [3, 17, 4], ix, ip)
    # position 3 -> page 7 slot 3; 17 -> page 2 slot 1; request 1 pos 4 -> page 4 slot 4
    assert torch.equal(out[7, 0, 3], k[0]) and torch.equal(out[7, 1, 3], v[0])
    assert torch.equal(out[2, 0, 1], k[1]) and torch.equal(out[4, 1, 4], v[2])
    changed = (out != pool).flatten(1).any(1).nonzero().flatten().tolist()
    assert changed == [2, 4, 7]
    kk, vv = opg.gather_kv(out, ip, ix, last, 0)
    assert kk.shape[0] == 20 and torch.equal(kk[17], k[1]) and torch.equal(vv[3], v[0])


def test_trace_admission_stops_at_first_misfit():
    t = opg.SchedulerTrace(4, 256, 16, max_num_pages=8)  # 7 free pages
    t.submit(opg.TraceRequest(0, 64, 10))   # 4 pages
    t.submit(opg.TraceRequest(1, 60, 10))   # 4 pages: does not fit -> stop
    t.submit(opg.TraceRequest(2, 10, 10))   # would fit, but FIFO blocks it
    r = t.step()
    assert [rid for rid, _ in r["admitted"]] == [0]
    assert len(t.waiting) == 2


def test_trace_growth_exhaustion_raises():
    """Decode growth is not admission-gated in the reference (843-847)."""
    t = opg.SchedulerTrace(2, 256, 16, max_num_pages=4)  # 3 free pages
    t.submit(opg.TraceRequest(0, 32, 40))  # 2 pages
    t.submit(opg.TraceRequest(1, 16, 40))  # 1 page; pool now empty
    with pytest.raises(RuntimeError):
        for _ in range(40):
            t.step()


def test_trace_invariants_random():
    rnd = random.Random(5)
    t = opg.SchedulerTrace(6, 512, 16, max_num_pages=120)
    for rid in range(50):
        t.submit(opg.TraceRequest(rid, rnd.randint(1, 200), rnd.randint(1, 30)))
    for _ in range(300):
        r = t.step()
        held = [p for q in t.active for p in q.pages]
        free = list(t.alloc.free_pages)
        # every page is either free or held exactly once; scratch never used
        assert sorted(held + free) == list(range(119))
        if r["decode"]:
            d = r["decode"]
            for i, pos in enumerate(d["positions"]):
                n = d["indptr"][i + 1] - d["indptr"][i]
                assert n == math.ceil((pos + 1) / 16)
