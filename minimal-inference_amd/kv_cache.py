"""Paged KV pool, the reference-compatible CSR builder, and the device page table.

Reference: PagedKVCache (scheduler.py:168-221), build_csr_metadata
(scheduler.py:267-302), the allocator call order of the step loop
(scheduler.py:596-600, 624-637, 843-847, 984-1003).

``PagedKVCache`` keeps the reference's surface (``kv_data[layer]`` views of
``[max_pages, 2, page_size, H_kv, D]``, ``scratch_page``, ``allocate_pages`` /
``release_pages``) but stores all layers in one allocation so a release can
zero a page in every layer with one kernel.

``DevicePageTable`` is the GPU replacement of the Python free list: the FIFO
ring and the per-slot page lists live in device memory and one kernel applies
a step's releases, admissions and decode growth and writes the CSR metadata.
The host keeps only counts, which follow from request lengths, so no step
reads device memory.
"""

from __future__ import annotations

import math
from collections import deque

import torch

from . import _lib
from ._util import require_gpu


class PagedKVCache:
    """All-layer KV pool ``[layers, max_pages, 2, page_size, H_kv, D]``."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, max_batch_size: int,
                 max_seq_len: int, page_size: int, device, dtype=torch.bfloat16,
                 max_num_pages: int | None = None):
        if dtype != torch.bfloat16:
            raise ValueError("the pool is bf16")
        self.page_size = page_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_pages_per_seq = math.ceil(max_seq_len / page_size)
        # scheduler.py:191-192 unless the caller sizes the pool explicitly
        self.max_num_pages = max_num_pages or max_batch_size * self.max_pages_per_seq
        self.data = torch.zeros(num_layers, self.max_num_pages, 2, page_size, num_kv_heads, head_dim,
                                dtype=dtype, device=device)
        self.kv_data = [self.data[i] for i in range(num_layers)]
        self.scratch_page = self.max_num_pages - 1  # scheduler.py:205
        # host FIFO (reference surface); the engine uses DevicePageTable instead
        self.free_pages: deque[int] = deque(range(self.max_num_pages - 1))

    @property
    def page_bytes(self) -> int:
        return 2 * self.page_size * self.num_kv_heads * self.head_dim * self.data.element_size()

    def allocate_pages(self, num_pages: int) -> list[int]:
        if len(self.free_pages) < num_pages:
            raise RuntimeError(f"Cannot allocate {num_pages} pages, only {len(self.free_pages)} free")
        return [self.free_pages.popleft() for _ in range(num_pages)]

    def release_pages(self, page_indices: list[int]) -> None:
        """Zero the pages in every layer (one kernel) and append them to the free list."""
        if page_indices:
            ids = torch.tensor(page_indices, dtype=torch.int32).to(self.data.device, non_blocking=True)
            self.zero_pages(ids, len(page_indices))
        self.free_pages.extend(page_indices)

    def zero_pages(self, page_ids: torch.Tensor, n: int) -> None:
        """Zero ``n`` pages (device int32 ids) in all layers."""
        if n == 0:
            return
        _lib.call("mi_pages_zero", self.data.data_ptr(), self.data[0].numel() * self.data.element_size(),
                  self.num_layers, self.max_num_pages, self.page_bytes, page_ids.data_ptr(), n,
                  torch.cuda.current_stream(self.data.device).cuda_stream)


def build_csr_metadata(page_lists: list[list[int]], seq_lens: list[int], page_size: int,
                       device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """scheduler.py:267-302: host page lists -> int32 indptr / indices / last_page_len.

    Kept for callers that hold page lists on the host; the engine builds the
    same arrays on the device with ``DevicePageTable.step``.
    """
    indptr = [0]
    flat: list[int] = []
    last: list[int] = []
    for pages, n in zip(page_lists, seq_lens):
        flat.extend(pages)
        indptr.append(len(flat))
        ln = n % page_size
        if ln == 0 and n > 0:
            ln = page_size
        last.append(ln)
    return (torch.tensor(indptr, dtype=torch.int32, device=device),
            torch.tensor(flat, dtype=torch.int32, device=device),
            torch.tensor(last, dtype=torch.int32, device=device))


class DevicePageTable:
    """FIFO free-page ring + per-slot page lists on the GPU.

    ``step()`` applies, in the reference's deque order, the releases queued by
    ``release()``, the admissions given, and decode growth, then writes CSR
    metadata for the given rows into caller buffers (e.g. a graph's static
    buffers).  Host-side counts mirror the device state exactly so admission
    and pool-exhaustion decisions never read the device.
    """

    def __init__(self, num_pages: int, max_slots: int, max_pages_per_slot: int, page_size: int, device):
        self.num_pages = num_pages
        self.max_slots = max_slots
        self.mpps = max_pages_per_slot
        self.page_size = page_size
        self.device = torch.device(device)
        nbytes = int(_lib.load().mi_page_table_state_size(num_pages, max_slots, max_pages_per_slot))
        if nbytes == 0:
            raise ValueError("bad page table geometry")
        self.state = torch.zeros((nbytes + 3) // 4, dtype=torch.int32, device=self.device)
        self._err_word = int(_lib.load().mi_page_table_error_offset(num_pages, max_slots, max_pages_per_slot)) // 4
        _lib.call("mi_page_table_init", self.state.data_ptr(), num_pages, max_slots, max_pages_per_slot,
                  torch.cuda.current_stream(self.device).cuda_stream)
        # host mirror
        self.free_count = num_pages - 1
        self.slot_npages = [0] * max_slots
        self._pending_release: list[int] = []
        self.released = torch.zeros(max(1, max_slots * max_pages_per_slot), dtype=torch.int32, device=self.device)
        # pinned staging for the per-step op list: a small ring, each slot
        # guarded by an event so a pending copy is never overwritten
        n_ops = 4 + 3 * max_slots + 2 * 1024
        self._ops_cpu = [torch.zeros(n_ops, dtype=torch.int32).pin_memory() for _ in range(4)]
        self._ops_evt = [None] * 4
        self._ops_i = 0
        self._ops_dev = torch.zeros(n_ops, dtype=torch.int32, device=self.device)

    @property
    def scratch_page(self) -> int:
        return self.num_pages - 1

    # ---------------------------------------------------------------- host mirror
    def pages_needed(self, seq_len: int) -> int:
        return math.ceil(seq_len / self.page_size)

    def can_admit(self, prompt_len: int) -> bool:
        return self.free_count >= self.pages_needed(prompt_len)

    def release(self, slot: int) -> None:
        """Release a slot's pages (scheduler.py:216-221).

        The host counts change at once, as the reference's deque does; the
        device ring receives the pages at the start of the next ``step()``,
        before that step's admissions, which is the same FIFO order.
        """
        self._pending_release.append((slot, self.slot_npages[slot]))
        self.free_count += self.slot_npages[slot]
        self.slot_npages[slot] = 0

    def error_word(self) -> int:
        """Sticky device error bits (synchronises; for tests and diagnostics)."""
        return int(self.state[self._err_word].item())

    # ---------------------------------------------------------------- device step
    def step(self, admits: list[tuple[int, int]], rows: list[tuple[int, int]], padded: int,
             indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
             batch_indices: torch.Tensor, positions: torch.Tensor, decode_plan=None) -> int:
        """One allocator + CSR step; returns the number of pages released.

        admits: (slot, npages) popped from the ring in order.
        rows:   (slot, position) of each batch row; a row grows its slot to
                ceil((position + 1) / page_size) pages and gets
                seq_len = position + 1.  Rows ``len(rows) .. padded-1`` own the
                scratch page only.
        decode_plan: optional (decode wrapper, num_qo_heads, num_kv_heads,
                head_dim): the wrapper is planned for the ``padded`` rows of
                this CSR in the same launch as the step (what
                ``wrapper.plan(indptr[:padded + 1], indices,
                last_page_len[:padded], ...)`` would do, without a second
                launch).
        Released pages are zeroed by the caller via ``released`` (the count is
        returned).
        """
        # Every check runs on prospective counts first; the host mirror (free
        # count, pages per slot, pending releases) changes only once the
        # step's kernel has been launched, so a step that raises leaves the
        # mirror equal to the device state.
        if padded < len(rows) or padded > 1024:
            raise ValueError("padded batch must be in [rows, 1024]")
        for name, t, n in (("indptr", indptr, padded + 1), ("last_page_len", last_page_len, padded),
                           ("batch_indices", batch_indices, padded), ("positions", positions, padded)):
            require_gpu(name, t)
            if t.dtype != torch.int32 or t.numel() < n:
                raise ValueError(f"{name} must be int32 with >= {n} entries")
        rel = [s for s, _ in self._pending_release]
        released_pages = sum(n for _, n in self._pending_release)
        n_rel = len(rel)
        free = self.free_count
        npages = {}  # slot -> prospective page count

        def held(s: int) -> int:
            return npages.get(s, self.slot_npages[s])

        for s, n in admits:
            if not 0 <= s < self.max_slots or n < 0:
                raise ValueError(f"bad admission (slot {s}, {n} pages)")
            if n > free:
                raise RuntimeError(f"Cannot allocate {n} pages, only {free} free")
            if held(s) + n > self.mpps:
                raise RuntimeError(f"slot {s} would exceed {self.mpps} pages")
            free -= n
            npages[s] = held(s) + n
        n_adm = len(admits)
        grow = 0
        for s, pos in rows:
            if not 0 <= s < self.max_slots or pos < 0:
                raise ValueError(f"bad decode row (slot {s}, position {pos})")
            need = self.pages_needed(pos + 1) - held(s)
            if need > 0:
                if held(s) + need > self.mpps:
                    raise RuntimeError(f"slot {s} would exceed {self.mpps} pages")
                grow += need
                npages[s] = held(s) + need
        if grow > free:
            raise RuntimeError(f"Cannot allocate {grow} pages, only {free} free")
        free -= grow
        total_pages = sum(held(s) for s, _ in rows) + (padded - len(rows))
        if total_pages > indices.numel():
            raise ValueError(f"indices buffer holds {indices.numel()} ids, step needs {total_pages}")
        ops = [n_rel, n_adm, len(rows), padded]
        ops += rel
        ops += [s for s, _ in admits]
        ops += [n for _, n in admits]
        ops += [s for s, _ in rows]
        ops += [p for _, p in rows]
        n = len(ops)
        k = self._ops_i
        self._ops_i = (k + 1) % len(self._ops_cpu)
        buf = self._ops_cpu[k]
        if n > buf.numel():
            raise ValueError("too many ops in one page-table step")
        if self._ops_evt[k] is not None:
            self._ops_evt[k].synchronize()  # the copy that last used this slot is done
        buf[:n] = torch.tensor(ops, dtype=torch.int32)
        self._ops_dev[:n].copy_(buf[:n], non_blocking=True)
        evt = torch.cuda.Event()
        evt.record(torch.cuda.current_stream(self.device))
        self._ops_evt[k] = evt
        stream = torch.cuda.current_stream(self.device).cuda_stream
        common = (self.state.data_ptr(), self.num_pages, self.max_slots, self.mpps, self._ops_dev.data_ptr(), n,
                  self.page_size, indptr.data_ptr(), indices.data_ptr(), indices.numel(), last_page_len.data_ptr(),
                  batch_indices.data_ptr(), positions.data_ptr(), self.released.data_ptr())
        if decode_plan is None:
            _lib.call("mi_page_table_step", *common, stream)
        else:
            wrapper, hq, hkv, d = decode_plan
            wrapper._check_plan_args(indptr, indices, last_page_len, hq, hkv)
            _lib.call("mi_page_table_step_decode_plan", *common, padded, wrapper._ws.data_ptr(), wrapper._ws_bytes,
                      hq, hkv, d, stream)
            wrapper._adopt_plan(indptr[: padded + 1], indices, last_page_len[:padded], hq, hkv, d, self.page_size)
        self._pending_release = []
        self.free_count = free
        for s, n in npages.items():
            self.slot_npages[s] = n
        return released_pages
