"""Paged KV pool, FIFO allocator replay, CSR metadata and append -- oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in plain Python / torch on the CPU:

* ``ReferenceAllocator`` -- PagedKVCache's free list (scheduler.py:168-221):
  ``max_pages = max_batch * ceil(max_seq / page_size)`` (191-192), the last
  page is the scratch page and the free deque starts as ``0 .. max_pages-2``
  (205-206), ``allocate`` pops from the left (208-214), ``release`` appends on
  the right (216-221).
* ``SchedulerTrace`` -- the allocator call order of the scheduler step
  (scheduler.py:596-600): admission in FIFO order, stopping at the first
  request that does not fit (624-637); decode growth before the step's
  metadata, in active-list order (843-847); release of finished requests at
  the end of the step, in active-list order (984-1003).
* ``build_csr`` -- build_csr_metadata (scheduler.py:267-302).
* ``decode_padding`` -- the graph padding of a decode batch
  (scheduler.py:887-896), with the padded rows given the scratch page.
* ``append`` -- append_paged_kv_cache slot placement (model.py:207-216, NHD
  layout scheduler.py:195-202).

Pinning: ``build_csr`` and ``append`` are pinned by closed-form invariants and
round trips in tests/test_oracle_paging.py; ``ReferenceAllocator`` and
``SchedulerTrace`` by hand-derived traces and FIFO invariants in the same file.
"""

from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass, field

import torch


class ReferenceAllocator:
    """FIFO free-page list of scheduler.py:168-221 (without the tensors)."""

    def __init__(self, max_num_pages: int):
        self.max_num_pages = max_num_pages
        self.scratch_page = max_num_pages - 1  # scheduler.py:205
        self.free_pages: deque[int] = deque(range(max_num_pages - 1))  # :206

    @classmethod
    def for_config(cls, max_batch_size: int, max_seq_len: int, page_size: int) -> "ReferenceAllocator":
        return cls(max_batch_size * math.ceil(max_seq_len / page_size))  # :191-192

    def allocate_pages(self, n: int) -> list[int]:
        if len(self.free_pages) < n:  # :210-213
            raise RuntimeError(f"Cannot allocate {n} pages, only {len(self.free_pages)} free")
        return [self.free_pages.popleft() for _ in range(n)]  # :214

    def release_pages(self, pages: list[int]) -> None:
        for p in pages:  # :218-221 (the zeroing is modelled by the pool oracle)
            self.free_pages.append(p)


def last_page_len(seq_len: int, page_size: int) -> int:
    """scheduler.py:293-296."""
    last = seq_len % page_size
    if last == 0 and seq_len > 0:
        last = page_size
    return last


def build_csr(page_lists: list[list[int]], seq_lens: list[int], page_size: int):
    """build_csr_metadata (scheduler.py:267-302) as int lists."""
    indptr = [0]
    flat: list[int] = []
    last: list[int] = []
    for pages, n in zip(page_lists, seq_lens):
        flat.extend(pages)
        indptr.append(len(flat))
        last.append(last_page_len(n, page_size))
    return indptr, flat, last


def decode_padding(indptr: list[int], indices: list[int], last: list[int], positions: list[int],
                   padded_batch: int, scratch_page: int):
    """Pad a decode batch to ``padded_batch`` rows.

    scheduler.py:887-896 repeats indptr's last value, sets last_page_len 1 and
    position 0 for padded rows and relies on the static index buffer holding
    the scratch page at ``indices[indptr[B]]`` (362-373).  Here each padded row
    owns exactly the scratch page, so its append provably lands there.
    """
    b = len(positions)
    indptr = list(indptr)
    indices = list(indices)
    last = list(last)
    positions = list(positions)
    for _ in range(padded_batch - b):
        indices.append(scratch_page)
        indptr.append(indptr[-1] + 1)
        last.append(1)
        positions.append(0)
    batch_indices = list(range(padded_batch))
    return indptr, indices, last, batch_indices, positions


@dataclass
class TraceRequest:
    rid: int
    prompt_len: int
    max_new_tokens: int
    pages: list[int] = field(default_factory=list)
    generated: int = 0
    position: int = 0
    admitted: bool = False
    finished: bool = False


class SchedulerTrace:
    """Replays the reference scheduler's page-allocation order for a trace.

    Tokens are not modelled: a request finishes after ``max_new_tokens``
    generated tokens (the first one comes from prefill, scheduler.py:741-751)
    or when its position reaches ``max_seq_len`` (972-973).
    """

    def __init__(self, max_batch_size: int, max_seq_len: int, page_size: int,
                 max_num_pages: int | None = None):
        self.page_size = page_size
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        n = max_num_pages or max_batch_size * math.ceil(max_seq_len / page_size)
        self.alloc = ReferenceAllocator(n)
        self.waiting: deque[TraceRequest] = deque()
        self.active: list[TraceRequest] = []

    def submit(self, req: TraceRequest) -> None:
        self.waiting.append(req)

    def step(self) -> dict:
        """One scheduler step; returns what the step did and the decode CSR."""
        out: dict = {"admitted": [], "released": [], "decode": None, "prefill": []}
        # admit (scheduler.py:624-637)
        newly = []
        while self.waiting and len(self.active) < self.max_batch_size:
            req = self.waiting[0]
            need = math.ceil(req.prompt_len / self.page_size)
            if len(self.alloc.free_pages) < need:
                break
            self.waiting.popleft()
            req.pages = self.alloc.allocate_pages(need)
            req.admitted = True
            self.active.append(req)
            newly.append(req)
            out["admitted"].append((req.rid, list(req.pages)))
        # prefill (scheduler.py:643-652, 741-751): first token, position = L;
        # finished when max_new_tokens is reached (no EOS in a trace).
        for req in newly:
            req.position = req.prompt_len
            req.generated = 1
            req.finished = req.generated >= req.max_new_tokens
            out["prefill"].append(req.rid)
        decoding = [r for r in self.active if not r.finished]
        # decode growth + CSR (scheduler.py:843-868), finish check (968-977)
        if decoding:
            for req in decoding:
                need = math.ceil((req.position + 1) / self.page_size)
                if need > len(req.pages):
                    req.pages.extend(self.alloc.allocate_pages(need - len(req.pages)))
            seq_lens = [r.position + 1 for r in decoding]
            indptr, indices, last = build_csr([r.pages for r in decoding], seq_lens, self.page_size)
            out["decode"] = {
                "rids": [r.rid for r in decoding],
                "positions": [r.position for r in decoding],
                "indptr": indptr,
                "indices": indices,
                "last_page_len": last,
            }
            for r in decoding:
                r.generated += 1
                r.position += 1
                r.finished = r.generated >= r.max_new_tokens or r.position >= self.max_seq_len
        # retire (scheduler.py:984-1003), in active-list order
        still = []
        for r in self.active:
            if r.finished:
                self.alloc.release_pages(r.pages)
                out["released"].append((r.rid, list(r.pages)))
            else:
                still.append(r)
        self.active = still
        return out


def append(pool: torch.Tensor, key: torch.Tensor, value: torch.Tensor, batch_indices, positions,
           indices, indptr) -> torch.Tensor:
    """append_paged_kv_cache slot placement (model.py:207-216) on a CPU copy.

    pool: [num_pages, 2, page_size, H_kv, D]; key/value: [T, H_kv, D].
    Rows whose page slot lies outside the request's page list are skipped,
    matching the library's documented contract.
    """
    pool = pool.clone()
    ps = pool.shape[2]
    bi = [int(x) for x in batch_indices]
    pos = [int(x) for x in positions]
    ind = [int(x) for x in indices]
    ptr = [int(x) for x in indptr]
    for i, (b, p) in enumerate(zip(bi, pos)):
        it = ptr[b] + p // ps
        if it >= ptr[b + 1]:
            continue
        page = ind[it]
        if not 0 <= page < pool.shape[0]:
            continue
        pool[page, 0, p % ps] = key[i]
        pool[page, 1, p % ps] = value[i]
    return pool


def gather_kv(pool: torch.Tensor, indptr, indices, last_page_len, b: int):
    """K and V of request b as [kv_len, H_kv, D] by walking its pages."""
    ps = pool.shape[2]
    lo, hi = int(indptr[b]), int(indptr[b + 1])
    n = hi - lo
    if n == 0:
        empty = pool.new_zeros((0,) + tuple(pool.shape[3:]))
        return empty, empty
    kv_len = (n - 1) * ps + int(last_page_len[b])
    pages = torch.as_tensor([int(x) for x in indices[lo:hi]], dtype=torch.long)
    sel = pool[pages]  # [n, 2, ps, H, D]
    k = sel[:, 0].reshape(n * ps, *pool.shape[3:])[:kv_len]
    v = sel[:, 1].reshape(n * ps, *pool.shape[3:])[:kv_len]
    return k, v
