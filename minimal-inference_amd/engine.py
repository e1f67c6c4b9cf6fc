"""Continuous-batching driver over the paged-attention path.

Restates the reference scheduler's semantics (scheduler.py:477-1009) on top
of the device page table and the HIP kernels:

* step order admit -> prefill -> decode -> retire (scheduler.py:596-600);
* admission in FIFO order while the batch has room, stopping at the first
  request whose ceil(len / page_size) pages do not fit (624-637);
* decode growth before the step's metadata, in active order (843-847);
* retirement at the end of the step releases pages in active order
  (984-1003); released pages are zeroed in every layer (216-221);
* greedy rows (temperature <= 0) take argmax, others sample (319-343).

What changes relative to the reference:
* page lists, the free-page ring and the CSR / padding metadata live on the
  GPU (``DevicePageTable``); the host keeps counts only;
* all requests admitted in a step are prefilled in one ragged batch (the
  reference prefills one request per forward, scheduler.py:643-652);
* the decode forward *and* the sampler are captured in one hipGraph per
  padded batch size; ``plan()`` runs outside the graph each step; padded rows
  own the scratch page, so their K/V appends land there by construction.

Per decode step the host performs one small host->device copy of op lists and
input ids, launches the page-table step (which plans the decode in the same
launch) and the graph, and reads the sampled ids back (needed to stream
tokens and detect EOS) -- once per window of ``decode_window`` steps (see
``_decode``).  With ``pipeline=True`` the next window is enqueued before the
host waits for the previous one's ids whenever the batch is unchanged, so
the GPU never idles while the host books tokens.  Every read-back also
carries the device page table's sticky error word and the decode plan's
error word; a nonzero one (host mirror and device state disagree, a plan
that did not fit) raises RuntimeError.

Serving: ``start()`` runs the step loop in a daemon thread and
``submit_request()`` hands requests to it from any thread
(scheduler.py:569-604); every token, then ``None`` once the request is
retired, goes to the request's ``sink`` (scheduler.py:1005-1009 pushes them
into the request's asyncio queue).
"""

from __future__ import annotations

import enum
import logging
import math
import threading
import time
from collections import deque
from dataclasses import dataclass, field
from typing import Callable

import torch

from .decode import BatchDecodeWithPagedKVCacheWrapper
from .kv_cache import DevicePageTable, PagedKVCache
from .model import AttentionBackend, Model
from .prefill import BatchPrefillWithPagedKVCacheWrapper
from .sampling import Sampler

GRAPH_BATCH_SIZES = [1, 2, 4, 8, 16, 32, 48, 64]  # scheduler.py:350


class RequestStatus(enum.Enum):
    WAITING = "waiting"
    PREFILLING = "prefilling"
    DECODING = "decoding"
    FINISHED = "finished"


@dataclass(eq=False)  # requests compare by identity (window membership, pipeline bookkeeping)
class Request:
    request_id: str
    input_ids: list[int]
    max_new_tokens: int
    temperature: float = 0.0
    top_p: float = 1.0
    status: RequestStatus = RequestStatus.WAITING
    generated_tokens: list[int] = field(default_factory=list)
    current_position: int = 0
    slot: int = -1
    finish_reason: str | None = None
    prefill_done_time: float = 0.0
    last_token_time: float = 0.0
    # receives each token id, then None when the request is retired
    sink: Callable[[int | None], None] | None = None


class _Pinned:
    """Pinned host staging buffer with an event guarding its last copy."""

    def __init__(self, n: int, dtype):
        self.buf = torch.zeros(n, dtype=dtype).pin_memory()
        self.evt: torch.cuda.Event | None = None

    def upload(self, values, dst: torch.Tensor) -> None:
        if self.evt is not None:
            self.evt.synchronize()
        n = len(values)
        self.buf[:n] = torch.as_tensor(values, dtype=self.buf.dtype)
        dst[:n].copy_(self.buf[:n], non_blocking=True)
        self.evt = torch.cuda.Event()
        self.evt.record()


@dataclass
class _Window:
    """A decode window enqueued on the GPU: its rows, length, pinned read-back
    slot, the event after its read-back, and its last step's sampled ids
    (a device tensor, the next window's input when the rows stay)."""

    members: list
    w: int
    slot: int
    evt: "torch.cuda.Event"
    last: torch.Tensor


class Scheduler:
    def __init__(self, model: Model, max_batch_size: int = 8, max_seq_len: int = 4096, page_size: int = 16,
                 num_pages: int | None = None, eos_token_ids: set[int] | None = None, use_graphs: bool = True,
                 seed: int = 0, workspace_mb: int = 128, zero_released_pages: bool = True, decode_window: int = 1,
                 keep_logits: bool = False, pipeline: bool = False):
        cfg = model.cfg
        self.model = model
        self.device = model.device
        self.page_size = page_size
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        self.eos = set(eos_token_ids or ())
        if decode_window < 1:
            raise ValueError("decode_window must be >= 1")
        self.decode_window = decode_window
        self.zero_released = zero_released_pages
        self.kv = PagedKVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, max_batch_size,
                               max_seq_len, page_size, self.device, max_num_pages=num_pages)
        mpps = math.ceil(max_seq_len / page_size) + 1
        self.pt = DevicePageTable(self.kv.max_num_pages, max_batch_size, mpps, page_size, self.device)
        dev = self.device
        ws = workspace_mb << 20
        self.decode_wrapper = BatchDecodeWithPagedKVCacheWrapper(torch.empty(ws, dtype=torch.uint8, device=dev))
        self.prefill_wrapper = BatchPrefillWithPagedKVCacheWrapper(torch.empty(ws, dtype=torch.uint8, device=dev))
        self.graph_sizes = [b for b in GRAPH_BATCH_SIZES if b < max_batch_size] + [max_batch_size]
        bmax = self.graph_sizes[-1]
        cap = bmax * mpps + bmax
        # static decode buffers (shared by every captured graph)
        self.d_indptr = torch.zeros(bmax + 1, dtype=torch.int32, device=dev)
        self.d_indices = torch.full((cap,), self.kv.scratch_page, dtype=torch.int32, device=dev)
        self.d_last = torch.ones(bmax, dtype=torch.int32, device=dev)
        self.d_batch = torch.arange(bmax, dtype=torch.int32, device=dev)
        self.d_pos = torch.zeros(bmax, dtype=torch.int32, device=dev)
        self.d_ids = torch.zeros(bmax, dtype=torch.int64, device=dev)
        self.sampler = Sampler(dev, bmax, seed=seed, vocab=cfg.vocab_size)
        # prefill buffers
        self.p_indptr = torch.zeros(max_batch_size + 1, dtype=torch.int32, device=dev)
        self.p_indices = torch.zeros(max_batch_size * mpps, dtype=torch.int32, device=dev)
        self.p_last = torch.ones(max_batch_size, dtype=torch.int32, device=dev)
        self.p_batch_dummy = torch.zeros(max_batch_size, dtype=torch.int32, device=dev)
        self.p_pos_dummy = torch.zeros(max_batch_size, dtype=torch.int32, device=dev)
        self.p_sampler = Sampler(dev, max_batch_size, seed=seed + 1, vocab=cfg.vocab_size)
        self._up_ids = _Pinned(bmax, torch.int64)
        self._up_t = _Pinned(bmax, torch.float32)
        self._up_p = _Pinned(bmax, torch.float32)
        self._tok_host = torch.zeros(max(bmax, max_batch_size), dtype=torch.int64).pin_memory()
        # decode window: sampled ids of every step of the window and, per row,
        # the first step whose id is an end-of-sequence id (computed on the GPU)
        self.d_ring = torch.zeros(decode_window, bmax, dtype=torch.int64, device=dev)
        self.d_eos = torch.tensor(sorted(self.eos) or [-1], dtype=torch.int64, device=dev)
        # two pinned read-back slots (a window's ids + first-EOS step per row),
        # so a window's copy never overwrites the one the host has not read;
        # per slot also the page table's error word and the plan's
        self._ring_host = [torch.zeros(decode_window + 1, bmax, dtype=torch.int64).pin_memory() for _ in range(2)]
        self._err_host = [torch.zeros(3, dtype=torch.int32).pin_memory() for _ in range(2)]
        self._slot = 0
        self.pipeline = pipeline
        self._inflight: _Window | None = None
        # keep_logits: the last decode step's logits [rows, V] (rows in the
        # decoding order of that step; copied inside the captured graphs) and
        # the last prefill's logits of each prompt's last token (admission order)
        self.keep_logits = keep_logits
        self.d_logits = torch.empty(bmax, cfg.vocab_size, dtype=model.dtype, device=dev) if keep_logits else None
        self.p_logits = torch.empty(max_batch_size, cfg.vocab_size, dtype=model.dtype, device=dev) \
            if keep_logits else None
        self.waiting: deque[Request] = deque()
        self.active: list[Request] = []
        self.free_slots: deque[int] = deque(range(max_batch_size))
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self.steps = 0
        # background loop state
        self._inbox: list[Request] = []
        self._aborts: set[str] = set()
        self._lock = threading.Lock()
        self._wake = threading.Event()
        self._running = False
        self._thread: threading.Thread | None = None
        self.loop_error: BaseException | None = None
        if use_graphs:
            self._capture_graphs()

    # ------------------------------------------------------------------ API
    def submit(self, req: Request) -> None:
        self.waiting.append(req)

    def has_work(self) -> bool:
        return bool(self.waiting or self.active)

    def run(self, max_steps: int | None = None) -> None:
        n = 0
        while self.has_work() and (max_steps is None or n < max_steps):
            self.step()
            n += 1
        self.flush()

    def flush(self) -> list[tuple[Request, int]]:
        """Read the decode window in flight (``pipeline``), book and push its
        tokens and retire the requests it finished."""
        if self._inflight is None:
            return []
        win, self._inflight = self._inflight, None
        emitted = self._collect(win)
        for r, t in emitted:
            self._push_token(r, t)
        self._retire()
        return emitted

    # ------------------------------------------------------------------ background loop
    def start(self) -> None:
        """Run the step loop in a daemon thread (scheduler.py:569-572)."""
        if self._thread is not None:
            raise RuntimeError("scheduler loop already started")
        self._running = True
        self._thread = threading.Thread(target=self._run_loop, name="mi-scheduler", daemon=True)
        self._thread.start()

    def stop(self) -> None:
        self._running = False
        self._wake.set()
        if self._thread is not None:
            self._thread.join()
            self._thread = None

    def submit_request(self, req: Request) -> None:
        """Thread-safe submit for a running loop (scheduler.py:580-584)."""
        if self.loop_error is not None:
            raise RuntimeError("scheduler loop stopped after an error") from self.loop_error
        n = len(req.input_ids)
        if n == 0 or n > self.max_seq_len:
            raise ValueError(f"prompt of {n} tokens (allowed 1..{self.max_seq_len})")
        if self.pt.pages_needed(n) > self.pt.num_pages - 1:
            raise ValueError(f"prompt of {n} tokens needs more pages than the pool holds")
        with self._lock:
            self._inbox.append(req)
        self._wake.set()

    def abort_request(self, request_id: str) -> None:
        """Thread-safe: stop a request of the running loop.  It finishes with
        finish_reason "abort" (its sink gets None) and its pages are released
        at the end of the loop's next step; unknown or finished ids are
        ignored."""
        with self._lock:
            self._aborts.add(request_id)
        self._wake.set()

    def _apply_aborts(self, ids: set[str]) -> None:
        kept = deque()
        for r in self.waiting:
            if r.request_id in ids:
                r.status = RequestStatus.FINISHED
                r.finish_reason = "abort"
                self._push_token(r, None)
            else:
                kept.append(r)
        self.waiting = kept
        for r in self.active:
            if r.request_id in ids and r.status != RequestStatus.FINISHED:
                r.status = RequestStatus.FINISHED  # retired (pages released, sink closed) by the next step
                r.finish_reason = "abort"

    def _run_loop(self) -> None:
        torch.cuda.set_device(self.device)
        while self._running:
            with self._lock:
                new, self._inbox = self._inbox, []
                aborts, self._aborts = self._aborts, set()
            for r in new:
                self.submit(r)
            if aborts:
                self._apply_aborts(aborts)
            if not self.has_work():
                self._wake.wait(timeout=0.1)
                self._wake.clear()
                continue
            try:
                self.step()
            except BaseException as e:  # fail every request, then stop
                logging.getLogger(__name__).exception("scheduler step failed")
                self.loop_error = e
                with self._lock:
                    pending, self._inbox = self._inbox, []
                for r in list(self.active) + list(self.waiting) + pending:
                    r.status = RequestStatus.FINISHED
                    r.finish_reason = "error"
                    self._push_token(r, None)
                self.active, self.waiting = [], deque()
                self._running = False

    @staticmethod
    def _push_token(req: Request, token: int | None) -> None:
        if req.sink is not None:
            req.sink(token)

    # ------------------------------------------------------------------ graphs
    def _backend(self, wrapper, mode, indptr, indices, last, batch, pos):
        return AttentionBackend(self.kv, wrapper, mode, indptr, indices, last, None, batch, pos)

    def _decode_forward(self, bs: int) -> torch.Tensor:
        be = self._backend(self.decode_wrapper, "decode", self.d_indptr[: bs + 1], self.d_indices,
                           self.d_last[:bs], self.d_batch[:bs], self.d_pos[:bs])
        logits = self.model.forward(self.d_ids[:bs], self.d_pos[:bs], be)
        if self.keep_logits:
            self.d_logits[:bs].copy_(logits)
        return self.sampler.sample(logits, bs, out=self.sampler.out[:bs])

    def _plan_decode(self, bs: int) -> None:
        cfg = self.model.cfg
        self.decode_wrapper.plan(self.d_indptr[: bs + 1], self.d_indices, self.d_last[:bs],
                                 cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.page_size)

    def _capture_graphs(self) -> None:
        for bs in self.graph_sizes:
            # all rows are padding rows: they own only the scratch page
            self.pt.step([], [], bs, self.d_indptr, self.d_indices, self.d_last, self.d_batch, self.d_pos)
            self._plan_decode(bs)
            self.sampler.temperature[:bs].fill_(0.0)
            s = torch.cuda.Stream(self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(s):
                for _ in range(2):
                    self._decode_forward(bs)
            torch.cuda.current_stream(self.device).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                out = self._decode_forward(bs)
            self.graphs[bs] = (g, out)
        torch.cuda.synchronize(self.device)

    # ------------------------------------------------------------------ step
    def step(self) -> list[tuple[Request, int]]:
        emitted: list[tuple[Request, int]] = []
        early: list[tuple[Request, int]] = []
        if (self.pipeline and self._inflight is not None and self.waiting
                and (self.eos or any(self._room(r) <= 0 for r in self._inflight.members))):
            # a request of the window in flight may end with it (its budget is
            # used up, or it may sample an end-of-sequence id): read the window
            # now, so a slot and pages it frees serve this step's admissions,
            # as in the unpipelined loop
            early = self.flush()
        admitted = self._admit()
        if admitted:
            emitted += self._prefill(admitted)
        decoding = [r for r in self.active if r.status == RequestStatus.DECODING]
        if decoding:
            emitted += self._decode(decoding)
        for r, t in emitted:
            self._push_token(r, t)
        self._retire()
        self.steps += 1
        return early + emitted

    def _admit(self) -> list[Request]:
        out = []
        while self.waiting and len(self.active) < self.max_batch_size:
            req = self.waiting[0]
            if len(req.input_ids) > self.max_seq_len:
                raise ValueError(f"prompt of {len(req.input_ids)} tokens exceeds max_seq_len {self.max_seq_len}")
            if not self.pt.can_admit(len(req.input_ids)):
                break
            self.waiting.popleft()
            req.slot = self.free_slots.popleft()
            req.status = RequestStatus.PREFILLING
            self.active.append(req)
            out.append(req)
        return out

    def _zero_released(self, n: int) -> None:
        if n and self.zero_released:
            self.kv.zero_pages(self.pt.released, n)

    def _prefill(self, reqs: list[Request]) -> list[tuple[Request, int]]:
        cfg = self.model.cfg
        dev = self.device
        admits = [(r.slot, self.pt.pages_needed(len(r.input_ids))) for r in reqs]
        rows = [(r.slot, len(r.input_ids) - 1) for r in reqs]
        n = len(reqs)
        released = self.pt.step(admits, rows, n, self.p_indptr, self.p_indices, self.p_last,
                                 self.p_batch_dummy, self.p_pos_dummy)
        self._zero_released(released)
        lens = [len(r.input_ids) for r in reqs]
        qo = [0]
        for x in lens:
            qo.append(qo[-1] + x)
        total = qo[-1]
        ids = torch.tensor([t for r in reqs for t in r.input_ids], dtype=torch.int64).to(dev, non_blocking=True)
        pos = torch.tensor([i for x in lens for i in range(x)], dtype=torch.int32).to(dev, non_blocking=True)
        bidx = torch.tensor([b for b, x in enumerate(lens) for _ in range(x)], dtype=torch.int32).to(dev, non_blocking=True)
        qo_d = torch.tensor(qo, dtype=torch.int32).to(dev, non_blocking=True)
        last_rows = (qo_d[1:] - 1).to(torch.int64)
        self.prefill_wrapper.plan(qo_d, self.p_indptr[: n + 1], self.p_indices, self.p_last[:n],
                                  cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.page_size,
                                  causal=True, max_total_q=total)
        be = self._backend(self.prefill_wrapper, "prefill", self.p_indptr[: n + 1], self.p_indices,
                           self.p_last[:n], bidx, pos)
        logits = self.model.forward(ids, pos, be, last_rows=last_rows)
        if self.keep_logits:
            self.p_logits[:n].copy_(logits)
        self.p_sampler.set_params([r.temperature for r in reqs], [r.top_p for r in reqs])
        toks = self.p_sampler.sample(logits, n)
        host = self._fetch(toks, n, self.prefill_wrapper._ws[4:8].view(torch.int32), "a prefill")
        now = time.perf_counter()
        out = []
        for r, t in zip(reqs, host):
            r.generated_tokens.append(t)
            r.current_position = len(r.input_ids)
            r.status = RequestStatus.DECODING
            r.prefill_done_time = r.last_token_time = now
            out.append((r, t))
            if t in self.eos or len(r.generated_tokens) >= r.max_new_tokens:
                r.status = RequestStatus.FINISHED
                r.finish_reason = "stop" if t in self.eos else "length"
        return out

    # ------------------------------------------------------------------ decode
    def in_flight(self, r: Request) -> int:
        """Tokens of ``r`` in the decode window in flight (enqueued, not yet
        read back; ``pipeline`` only)."""
        w = self._inflight
        return w.w if w is not None and r in w.members else 0

    def _room(self, r: Request) -> int:
        """Tokens ``r`` may still be given beyond those already enqueued."""
        pend = self.in_flight(r)
        return min(r.max_new_tokens - len(r.generated_tokens) - pend,
                   self.max_seq_len - (r.current_position + pend))

    def _decode(self, reqs: list[Request]) -> list[tuple[Request, int]]:
        """Decode W = min(decode_window, tokens any request may still take)
        steps with one host round trip.  Within the window the sampled ids are
        fed back on the GPU (scheduler.py:962-978 does it on the host per
        step), each step's page-table step and plan run ahead without waiting,
        and end-of-sequence detection runs on the GPU over the window's ids.
        A row that samples an end-of-sequence id keeps decoding to the end of
        the window (its extra tokens are dropped, its pages freed at retire).

        Without ``pipeline`` the window's ids are read back before returning.
        With it, a window whose rows are the window in flight's is enqueued
        first (its input ids are the last sampled ids, still on the GPU), then
        the window in flight is read: the call returns that window's tokens,
        one window late.  When the rows differ (an admission, a retirement,
        a request out of budget) the window in flight is read first."""
        if not self.pipeline:
            return self._collect(self._enqueue_window(reqs, None))
        emitted: list[tuple[Request, int]] = []
        cand = [r for r in reqs if self._room(r) > 0]
        prev = self._inflight
        if prev is not None and cand == prev.members:
            self._inflight = self._enqueue_window(cand, prev)
            return self._collect(prev)
        if prev is not None:
            self._inflight = None
            emitted += self._collect(prev)
            cand = [r for r in self.active if r.status == RequestStatus.DECODING and self._room(r) > 0]
        if cand:
            self._inflight = self._enqueue_window(cand, None)
        return emitted

    def _enqueue_window(self, reqs: list[Request], prev: "_Window | None") -> "_Window":
        """Enqueue one window of decode steps for ``reqs`` and its read-back
        into a pinned slot (nothing waits here).  With ``prev`` (the window in
        flight over the same rows) the first step's input ids are prev's last
        sampled ids, taken on the GPU."""
        b = len(reqs)
        bs = next((g for g in self.graph_sizes if g >= b), None)
        graph = self.graphs.get(bs) if bs is not None else None
        padded = bs if graph is not None else b
        if padded > self.d_batch.numel():
            raise RuntimeError(f"decode batch {b} exceeds the static buffers ({self.d_batch.numel()})")
        start = [r.current_position + self.in_flight(r) for r in reqs]
        w = min([self.decode_window] + [self._room(r) for r in reqs])
        w = max(1, w)
        # shrink the window until the pool covers every row's growth over it
        # (one step that does not fit raises, as allocate_pages does)
        while w > 1 and sum(max(0, self.pt.pages_needed(p + w) - self.pt.slot_npages[r.slot])
                            for r, p in zip(reqs, start)) > self.pt.free_count:
            w -= 1
        if prev is None:
            self._up_t.upload([r.temperature for r in reqs] + [0.0] * (padded - b), self.sampler.temperature)
            self._up_p.upload([r.top_p for r in reqs] + [1.0] * (padded - b), self.sampler.top_p)
        cfg = self.model.cfg
        plan = (self.decode_wrapper, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim)
        toks = prev.last if prev is not None else None
        for j in range(w):
            rows = [(r.slot, p + j) for r, p in zip(reqs, start)]
            # page-table step and the decode plan of its rows: one launch
            released = self.pt.step([], rows, padded, self.d_indptr, self.d_indices, self.d_last, self.d_batch,
                                    self.d_pos, decode_plan=plan)
            self._zero_released(released)
            if toks is None:
                self._up_ids.upload([r.generated_tokens[-1] for r in reqs] + [0] * (padded - b), self.d_ids)
            else:
                self.d_ids[:padded].copy_(toks[:padded])
            if graph is not None:
                g, out = graph
                g.replay()
                toks = out
            else:
                toks = self._decode_forward(padded)
            if w > 1:
                self.d_ring[j, :padded].copy_(toks[:padded])
        k = self._slot
        self._slot ^= 1
        host = self._ring_host[k]
        if w == 1:
            host[0, :b].copy_(toks[:b], non_blocking=True)
        else:
            ring = self.d_ring[:w, :b]
            hit = torch.isin(ring, self.d_eos)
            first = torch.where(hit.any(0), hit.to(torch.int8).argmax(0), torch.full_like(ring[0], w))
            host[:w, :b].copy_(ring, non_blocking=True)
            host[w, :b].copy_(first, non_blocking=True)
        # the page table's sticky word also holds every step's plan error
        err = self._err_host[k]
        err[0:1].copy_(self.pt.state[self.pt._err_word: self.pt._err_word + 1], non_blocking=True)
        err[1] = 0
        evt = torch.cuda.Event()
        evt.record(torch.cuda.current_stream(self.device))
        return _Window(list(reqs), w, k, evt, toks)

    def _check_errors(self, err: list[int], what: str) -> None:
        if err[0] & 0xFF:
            raise RuntimeError(f"device page table error bits {err[0]:#x} after {what}: the host's page counts and "
                               f"the device state disagree (1 release, 2 admission, 4 growth, 8 indices capacity, "
                               f"16 malformed ops)")
        if err[0] >> 8:
            raise RuntimeError(f"{what}: decode plan error bits {err[0] >> 8} in a step's fused plan (1: work items "
                               f"did not fit the workspace, 2: the page-table step before it failed)")
        if err[1]:
            raise RuntimeError(f"{what}: plan error {err[1]} (1: work items did not fit the workspace, 2: the "
                               f"page-table step before it failed)")

    def _collect(self, win: "_Window") -> list[tuple[Request, int]]:
        """Wait for a window's read-back, check the device error words, book
        its tokens (requests finished before it keep none)."""
        win.evt.synchronize()
        self._check_errors(self._err_host[win.slot].tolist(), "a decode window")
        w, reqs = win.w, win.members
        b = len(reqs)
        host = self._ring_host[win.slot][: w + 1, :b].tolist()
        if w == 1:
            host_rows = [[host[0][i]] for i in range(b)]
            stops = [0 if row[0] in self.eos else 1 for row in host_rows]
        else:
            host_rows = [[host[j][i] for j in range(w)] for i in range(b)]
            stops = host[w]
        now = time.perf_counter()
        out_list = []
        for i, r in enumerate(reqs):
            if r.status != RequestStatus.DECODING:
                continue  # finished (end of sequence) in an earlier window
            take = min(w, stops[i] + 1) if stops[i] < w else w
            for t in host_rows[i][:take]:
                r.generated_tokens.append(t)
                r.current_position += 1
                r.last_token_time = now
                out_list.append((r, t))
                if t in self.eos or len(r.generated_tokens) >= r.max_new_tokens or \
                        r.current_position >= self.max_seq_len:
                    r.status = RequestStatus.FINISHED
                    r.finish_reason = "stop" if t in self.eos else "length"
                    break
            if r.status != RequestStatus.FINISHED and take < w:
                raise AssertionError("decode window stopped early without an end-of-sequence id")
        return out_list

    def _fetch(self, toks: torch.Tensor, n: int, ws_err: torch.Tensor | None = None, what: str = "") -> list[int]:
        """Read ``n`` sampled ids back (one wait), with the page table's error
        word and, given ``ws_err`` (a device int32 word), a plan's."""
        self._tok_host[:n].copy_(toks[:n], non_blocking=True)
        err = self._err_host[self._slot]
        err[0:1].copy_(self.pt.state[self.pt._err_word: self.pt._err_word + 1], non_blocking=True)
        if ws_err is not None:
            err[1:2].copy_(ws_err, non_blocking=True)
        else:
            err[1] = 0
        torch.cuda.current_stream(self.device).synchronize()
        self._check_errors(err.tolist(), what)
        return self._tok_host[:n].tolist()

    def _retire(self) -> None:
        still = []
        for r in self.active:
            if r.status == RequestStatus.FINISHED:
                self.pt.release(r.slot)
                self.free_slots.append(r.slot)
                self._push_token(r, None)
            else:
                still.append(r)
        self.active = still
