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


def _plan_bytes(ws: torch.Tensor) -> torch.Tensor:
    """The part of a decode workspace a plan writes and a run only reads: the
    256-byte header and the work items (128 bytes each, header word 1 counts
    them).  The rest is the run's scratch (split partials), which the plan
    does not write."""
    n_items = int(ws[:16].view(torch.int32)[1])
    return ws[: 256 + 128 * n_items]


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


def test_padded_batch_of_1024_writes_every_indptr_entry(dev):
    """padded == 1024 (one row per thread of the page-table kernel): the
    1,025th indptr entry must be written too, against the oracle CSR."""
    from minimal_inference_amd.kv_cache import DevicePageTable

    n_rows, padded = 1000, 1024
    pt = DevicePageTable(4096, n_rows, 4, 16, dev)
    indptr = torch.full((padded + 1,), -7, dtype=torch.int32, device=dev)
    indices = torch.full((padded * 4,), -7, dtype=torch.int32, device=dev)
    last = torch.zeros(padded, dtype=torch.int32, device=dev)
    bidx = torch.zeros(padded, dtype=torch.int32, device=dev)
    pos = torch.zeros(padded, dtype=torch.int32, device=dev)
    lens = [1 + (7 * i) % 40 for i in range(n_rows)]  # 1..40 tokens: 1..3 pages
    admits = [(i, pt.pages_needed(n)) for i, n in enumerate(lens)]
    pt.step(admits, [], 0, indptr, indices, last, bidx, pos)
    rows = [(i, n - 1) for i, n in enumerate(lens)]
    pt.step([], rows, padded, indptr, indices, last, bidx, pos)
    npages = [pt.pages_needed(n) for n in lens] + [1] * (padded - n_rows)
    want = [0]
    for n in npages:
        want.append(want[-1] + n)
    got = indptr.cpu().tolist()
    assert got == want
    # real rows got consecutive ring pages in admission order, padding rows the scratch page
    ix = indices[: want[-1]].cpu().tolist()
    assert ix[: want[n_rows]] == list(range(want[n_rows]))
    assert ix[want[n_rows]:] == [4095] * (padded - n_rows)
    assert pt.error_word() == 0


def test_failed_step_leaves_the_host_mirror_unchanged(dev):
    """A step that raises before its launch must not move the host counts:
    the device never saw it, so free_count / pages per slot / pending
    releases stay as they were and the next step still matches the oracle."""
    from minimal_inference_amd.kv_cache import DevicePageTable

    pt = DevicePageTable(40, 4, 8, 16, dev)
    buf = [torch.zeros(16, dtype=torch.int32, device=dev) for _ in range(5)]
    pt.step([(0, 2), (1, 3)], [], 0, *buf)
    pt.release(1)
    before = (pt.free_count, list(pt.slot_npages), list(pt._pending_release))
    small = torch.zeros(2, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):  # indices buffer too small for the step's pages
        pt.step([(2, 5)], [(0, 40), (2, 70)], 2, buf[0], small, buf[2], buf[3], buf[4])
    with pytest.raises(ValueError):  # padded batch below the row count
        pt.step([(2, 1)], [(0, 20), (2, 3)], 1, *buf)
    with pytest.raises(RuntimeError):  # admission beyond the pool
        pt.step([(2, 9), (3, 30)], [], 0, *buf)
    assert (pt.free_count, pt.slot_npages, pt._pending_release) == before
    # the real step: release of slot 1 (3 pages to the ring tail), then growth of slot 0
    pt.step([], [(0, 40)], 1, *buf)
    assert buf[0][:2].cpu().tolist() == [0, 3]
    assert buf[1][:3].cpu().tolist() == [0, 1, 5]
    assert pt.free_count == 39 - 3
    assert pt.error_word() == 0


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (28, 4, 128)])
def test_fused_step_and_plan_equal_step_then_plan(dev, hq, hkv, d):
    """mi_page_table_step_decode_plan (one launch) writes the CSR that
    mi_page_table_step writes and the decode workspace that mi_decode_plan
    then writes (header and work items), byte for byte, over steps with
    admissions, growth, releases and graph padding; the decode attention run
    on either plan is identical."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    from minimal_inference_amd.kv_cache import DevicePageTable

    ps, max_bs, mpps, num_pages = 16, 40, 80, 3000
    rng = random.Random(hq * 100 + d)
    tables, bufs, wrappers = [], [], []
    for _ in range(2):
        tables.append(DevicePageTable(num_pages, max_bs, mpps, ps, dev))
        bufs.append([torch.zeros(n, dtype=torch.int32, device=dev)
                     for n in (max_bs + 1, max_bs * mpps + 64, max_bs, max_bs, max_bs)])
        wrappers.append(BatchDecodeWithPagedKVCacheWrapper(torch.zeros(64 << 20, dtype=torch.uint8, device=dev)))
    pool = torch.randn(num_pages, 2, ps, hkv, d, device=dev).to(torch.bfloat16)
    pos = {}
    free_slots = list(range(max_bs))
    for step in range(12):
        admits = []
        for _ in range(rng.randint(0, 6) if step else 24):
            if not free_slots:
                break
            s = free_slots.pop(0)
            n = rng.randint(1, 500)
            admits.append((s, math.ceil(n / ps)))
            pos[s] = n - 1
        if step % 3 == 2:  # retire a few
            for s in rng.sample(sorted(pos), k=min(3, len(pos))):
                for pt in tables:
                    pt.release(s)
                del pos[s]
                free_slots.append(s)
        for s in pos:
            pos[s] += rng.randint(0, 20)
        rows = [(s, p) for s, p in sorted(pos.items())]
        padded = next(g for g in (1, 2, 4, 8, 16, 32, 40) if g >= len(rows))
        tables[0].step(admits, rows, padded, *bufs[0])
        wrappers[0].plan(bufs[0][0][: padded + 1], bufs[0][1], bufs[0][2][:padded], hq, hkv, d, ps)
        tables[1].step(admits, rows, padded, *bufs[1], decode_plan=(wrappers[1], hq, hkv, d))
        torch.cuda.synchronize()
        for a, b in zip(bufs[0], bufs[1]):
            assert torch.equal(a, b), step
        assert torch.equal(_plan_bytes(wrappers[0]._ws), _plan_bytes(wrappers[1]._ws)), step
        q = torch.randn(padded, hq, d, device=dev).to(torch.bfloat16)
        assert torch.equal(wrappers[0].run(q, pool), wrappers[1].run(q, pool)), step
    assert tables[0].error_word() == 0 and tables[1].error_word() == 0


@pytest.mark.parametrize("n_rows,padded,row_pages,hq,hkv,d", [
    (100, 128, 3, 32, 8, 128),    # 65..1024 rows: the block-wide search and item writer
    (1000, 1024, 2, 14, 2, 64),   # the largest padded batch, page ids on chip
    (1000, 1024, 12, 32, 8, 128),  # a CSR of 12,000+ pages, over the 8,192 kept on chip
])
def test_fused_step_and_plan_large_batches(dev, n_rows, padded, row_pages, hq, hkv, d):
    """The fused step + plan on padded batches above 64 rows (the plan's
    block-wide search over on-chip row data) and on a CSR too large for the
    on-chip copy of its page ids (the items then read the indices the same
    workgroup has just written): CSR buffers, the decode workspace and the
    attention run equal mi_page_table_step followed by mi_decode_plan."""
    from minimal_inference_amd.decode import BatchDecodeWithPagedKVCacheWrapper
    from minimal_inference_amd.kv_cache import DevicePageTable

    ps, mpps = 16, row_pages + 2
    num_pages = n_rows * (row_pages + 1) + 64
    rng = random.Random(n_rows + row_pages)
    lens = [rng.randint((row_pages - 1) * ps + 1, row_pages * ps) for _ in range(n_rows)]
    tables, bufs, wrappers = [], [], []
    for _ in range(2):
        tables.append(DevicePageTable(num_pages, n_rows, mpps, ps, dev))
        bufs.append([torch.zeros(n, dtype=torch.int32, device=dev)
                     for n in (padded + 1, padded * mpps + 64, padded, padded, padded)])
        wrappers.append(BatchDecodeWithPagedKVCacheWrapper(torch.zeros(64 << 20, dtype=torch.uint8, device=dev)))
    admits = [(i, math.ceil(n / ps)) for i, n in enumerate(lens)]
    for pt, b in zip(tables, bufs):
        pt.step(admits, [], 0, *b)
    # one decode step at position len (growth into a new page for the rows whose prompt filled theirs)
    rows = [(i, n) for i, n in enumerate(lens)]
    tables[0].step([], rows, padded, *bufs[0])
    wrappers[0].plan(bufs[0][0][: padded + 1], bufs[0][1], bufs[0][2][:padded], hq, hkv, d, ps)
    tables[1].step([], rows, padded, *bufs[1], decode_plan=(wrappers[1], hq, hkv, d))
    torch.cuda.synchronize()
    total = int(bufs[0][0][padded])
    assert total >= n_rows * row_pages
    if row_pages == 12:
        assert total > 8192
    for a, b in zip(bufs[0], bufs[1]):
        assert torch.equal(a, b)
    assert torch.equal(_plan_bytes(wrappers[0]._ws), _plan_bytes(wrappers[1]._ws))
    pool = torch.randn(num_pages, 2, ps, hkv, d, device=dev).to(torch.bfloat16)
    q = torch.randn(padded, hq, d, device=dev).to(torch.bfloat16)
    assert torch.equal(wrappers[0].run(q, pool), wrappers[1].run(q, pool))
    assert tables[0].error_word() == 0 and tables[1].error_word() == 0
