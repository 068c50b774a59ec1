"""Continuous-batching scheduler driving the paged KV pool — drop-in for
muserve/scheduler.py.

``ContinuousBatchScheduler`` keeps the reference's class, request type and
methods (muserve/scheduler.py:22-123): ``add_request``, ``schedule_step``
(decode every running request, admit waiting ones while running + admitted <
max_batch_size), ``finish_prefill``, ``finish_request`` and the counters, with
the same semantics.

Attached to a ``PagedKVCache`` it also plans whole steps for the pool:

* ``plan_step()`` decodes every running request (one token each) and spends a
  prefill budget of ``chunked_prefill_size`` tokens (muserve/config.py:40) on
  requests being prefilled, oldest first, then on newly admitted ones. A
  request takes as many prompt tokens as the budget and the free pages allow;
  the first request that gets none ends the step's prefill. Pages come from
  the pool's LIFO free list in the order repeated ``alloc_pages(1)`` calls
  would give them (decode entries first, then the chunks). An admitted
  request takes the smallest free batch row, which is also its GDN state slot
  (with ``state_pool=``, ``launch_plan`` zeroes an admitted request's slots in
  every layer).
* One ``mkv_step_plan`` launch then writes the step's slot mapping, positions,
  cu_seqlens, per-entry block tables (``to_page_table_tensor`` layout:
  pages, then zeros), sequence lengths and rows on the device. The host only
  uploads one small record per entry plus the new page ids; no per-token work
  runs on the host.
* ``complete_step(plan, tokens)`` applies the sampled tokens: a decode entry
  appends its token; a chunk that finished its prompt appends the first token
  and joins the running batch (``finish_prefill``); a request finishes at
  ``max_new_tokens``, on ``eos_token_id``, or when its next decode would pass
  ``max_seq_len`` (``finish_request``). Its pages and row are freed at the
  next ``plan_step``.

With a ``BlockManager`` attached (``block_manager=``), admissions reuse
cached prompt pages. The block manager owns pool pages [0, its num_pages)
(taken out of the cache's free list); the cache's free list keeps the rest
for each request's private pages. A request's shareable pages are the full
pages before its last prompt token, fb = (n - 1) // 16. Its admission hashes
them on the GPU (``mkv_block_hash_sha256``) and admits them through
``mkv_bm_step`` (leading cached pages shared and pinned, the others taken from
the block manager's free stack or by evicting its least recently released
cached page, their hashes registered); the chunked prefill then starts at its
first uncached page, and its tail page (the page of its last prompt token,
where decoding continues) and decode pages come from the private list. A
finished request's release returns its cached pages to the block manager's
LRU instead of a free list. Admission candidates are the queue's head while
the budget, counted as if nothing were cached, is not spent, a row and a
private page are free; the block manager's work for a step (releases, then
the candidates' admits) runs on a side stream, and the host waits for its
results (hits and page ids) before it plans the chunks: it reads them right
after the many-CU passes when those committed every admit (the usual case),
and otherwise after the one-workgroup kernels. ``oracle/sched.py``
(``PrefixSchedulerModel``) states the policy.

Entries are ordered decode tokens first (running order), then prefill chunks,
so ``plan.block_tables[:plan.num_decode]`` and ``plan.seq_lens[:plan.num_decode]``
are what ``attn_decode`` reads for the decode half. A plan's device tensors
are rewritten by the next ``plan_step``: work that reads them must be issued
on the same stream before then (stream order does the rest).
"""
from __future__ import annotations

import heapq
import threading
import time
from collections import deque
from dataclasses import dataclass, field
from enum import Enum
from typing import Optional

import numpy as np
import torch

from muserve_amd import _lib
from muserve_amd.config import CHUNKED_PREFILL_SIZE, KV_PAGE_SIZE
from muserve_amd.kv_cache import PagedKVCache, SequenceKVState
from muserve_amd.memory.kv_cache import KVCache

_ENTRY_INTS = 8  # MkvStepEntry: row, start, count, held, new_pages, page_off, tok_off, reserved


class RequestState(Enum):
    WAITING = "waiting"
    PREFILLING = "prefilling"
    DECODING = "decoding"
    FINISHED = "finished"


@dataclass
class InferenceRequest:
    """muserve/scheduler.py:29-51, plus the paged-pool bookkeeping."""
    request_id: str
    input_ids: list[int]
    max_new_tokens: int = 256
    temperature: float = 0.0
    state: RequestState = RequestState.WAITING
    generated_tokens: list[int] = field(default_factory=list)
    gdn_states: Optional[list] = None
    kv_cache: Optional[KVCache] = None
    created_at: float = field(default_factory=time.time)
    first_token_at: Optional[float] = None
    finished_at: Optional[float] = None
    # paged pool: the sequence's pages and length, its batch row (also its
    # GDN state slot) and how much of the prompt is in the cache
    seq: Optional[SequenceKVState] = None
    row: int = -1
    num_prefilled: int = 0
    # prefix reuse: shareable pages (held by the block manager), how many of
    # them were cache hits, and how many of the row's pages the device table
    # holds
    fb: int = 0
    hits: int = 0
    dev_held: int = 0
    bm_id: int = -1  # its request id in the block manager
    page_hashes: Optional[torch.Tensor] = field(default=None, repr=False)  # until admitted

    @property
    def total_len(self) -> int:
        return len(self.input_ids) + len(self.generated_tokens)

    @property
    def is_done(self) -> bool:
        return self.state == RequestState.FINISHED


@dataclass
class StepPlan:
    """One scheduled step. Host lists describe the entries; the tensors are
    device views written by ``mkv_step_plan`` (valid until the next plan)."""
    decode: list[InferenceRequest]
    prefill: list[tuple[InferenceRequest, int, int]]  # (request, start, count)
    num_tokens: int
    upload: np.ndarray                  # what the kernel read: entries, then new pages
    slot_mapping: torch.Tensor          # [num_tokens] int64
    positions: torch.Tensor             # [num_tokens] int64
    cu_seqlens: torch.Tensor            # [num_entries + 1] int64
    block_tables: torch.Tensor          # [num_entries, width] int32
    seq_lens: torch.Tensor              # [num_entries] int32, after the step
    rows: torch.Tensor                  # [num_entries] int32 batch rows / GDN state slots
    admitted: list[InferenceRequest] = field(default_factory=list)  # admitted this step
    fresh: list[int] = field(default_factory=list)  # entries whose request starts here
    skipped_tokens: int = 0             # prompt tokens found in the prefix cache this step
    bm_ops: list[int] = field(default_factory=list)  # block-manager ops of this step

    @property
    def num_decode(self) -> int:
        return len(self.decode)

    @property
    def num_entries(self) -> int:
        return len(self.decode) + len(self.prefill)

    @property
    def entries(self) -> list[InferenceRequest]:
        return self.decode + [r for r, _, _ in self.prefill]


class ContinuousBatchScheduler:
    """Continuous batching scheduler (muserve/scheduler.py:54-123) with a paged
    step planner when a ``PagedKVCache`` is attached."""

    _RING = 4  # pinned upload buffers in flight

    def __init__(self, max_batch_size: int = 8, max_seq_len: int = 32768,
                 device: torch.device = None, *, kv_cache: PagedKVCache | None = None,
                 chunked_prefill_size: int = CHUNKED_PREFILL_SIZE,
                 eos_token_id: int | None = None, state_pool=None, block_manager=None):
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        self.device = device

        self.waiting_queue: deque[InferenceRequest] = deque()
        self.running_batch: list[InferenceRequest] = []
        self.lock = threading.Lock()

        self.kv_cache = kv_cache
        self.chunked_prefill_size = chunked_prefill_size
        self.eos_token_id = eos_token_id
        self.prefilling: list[InferenceRequest] = []
        self._free_rows = list(range(max_batch_size))
        self.width = -(-max_seq_len // KV_PAGE_SIZE)  # pages per row
        self._last: StepPlan | None = None
        self._dev = None
        # GDN state pool indexed by batch row: an admitted request's slots are
        # zeroed in every layer by launch_plan
        if state_pool is not None and state_pool.num_slots < max_batch_size:
            raise ValueError(f"state pool has {state_pool.num_slots} slots for "
                             f"{max_batch_size} batch rows")
        if state_pool is not None and block_manager is not None:
            # a prefix hit skips prefill of the hit pages, but the GDN layers'
            # recurrent and conv states at the end of that prefix are not
            # cached (the reference keeps them with each prefix entry,
            # muserve/model/prefix_cache.py:74-79,98-105): the request would
            # start its recurrent layers from zero states partway through its
            # prompt. Prefix reuse is therefore for attention-only stacks.
            raise ValueError("prefix reuse (block_manager=) does not cache GDN states: it "
                             "cannot be combined with a state_pool")
        self.state_pool = state_pool
        self.block_manager = block_manager
        self.bm_held = 0          # sum of fb over requests admitted to the block manager
        self.prefix_skipped = 0   # prompt tokens served from cached pages so far
        if block_manager is not None:
            if kv_cache is None:
                raise ValueError("prefix reuse needs the paged pool (kv_cache=...)")
            bm = block_manager
            if bm.device != kv_cache.device or bm.num_pages > kv_cache.num_pages:
                raise ValueError("the block manager must own a page range of the cache's pool")
            if bm.tables.shape[0] != 2 * max_batch_size or bm.tables.shape[1] < self.width:
                raise ValueError(f"the block manager needs {2 * max_batch_size} requests (twice "
                                 f"the batch) and >= {self.width} pages per request")
            kv_cache.reserve_range(0, bm.num_pages)
            # block-manager request ids: a FIFO of twice the batch, so an id
            # released in a step is not admitted again in that step (an admit
            # takes the front, a release appends); each id's length stays
            # until its release, which reads it
            self._bm_ids = deque(range(2 * max_batch_size))
            self._unhashed: list[InferenceRequest] = []  # queued, page hashes not yet launched
            self._bm_ntok = np.zeros(2 * max_batch_size, dtype=np.int64)
            # rounds whose results were read after the many-CU half / after
            # the one-workgroup kernels
            self.bm_early_rounds = self.bm_late_rounds = 0
        if kv_cache is not None:
            if chunked_prefill_size <= 0:
                raise ValueError("chunked_prefill_size must be positive")
            if kv_cache.device.type == "cuda":
                self._alloc_device(kv_cache.device)

    # ── reference protocol (muserve/scheduler.py:69-123) ────────────────────

    def add_request(self, request: InferenceRequest):
        if self.kv_cache is not None:
            n = len(request.input_ids)
            if n == 0:
                raise ValueError(f"request {request.request_id}: empty prompt")
            if n > self.max_seq_len:
                raise ValueError(f"request {request.request_id}: prompt of {n} tokens exceeds "
                                 f"max_seq_len {self.max_seq_len}")
        with self.lock:
            self.waiting_queue.append(request)
            if self.block_manager is not None:
                self._unhashed.append(request)

    def schedule_step(self) -> tuple[list[InferenceRequest], list[InferenceRequest]]:
        """(prefill_requests, decode_requests): drop finished requests, decode
        every running one, admit waiting ones while the batch has room."""
        with self.lock:
            self.running_batch = [r for r in self.running_batch if not r.is_done]
            decode_requests = list(self.running_batch)
            prefill_requests = []
            while (self.waiting_queue
                   and len(self.running_batch) + len(prefill_requests) < self.max_batch_size):
                req = self.waiting_queue.popleft()
                req.state = RequestState.PREFILLING
                prefill_requests.append(req)
            return prefill_requests, decode_requests

    def finish_prefill(self, requests: list[InferenceRequest]):
        with self.lock:
            for req in requests:
                req.state = RequestState.DECODING
                req.first_token_at = time.time()
                self.running_batch.append(req)

    def finish_request(self, request: InferenceRequest):
        request.state = RequestState.FINISHED
        request.finished_at = time.time()

    @property
    def num_waiting(self) -> int:
        return len(self.waiting_queue)

    @property
    def num_running(self) -> int:
        return len(self.running_batch)

    @property
    def num_prefilling(self) -> int:
        return len(self.prefilling)

    @property
    def is_idle(self) -> bool:
        return self.num_waiting == 0 and self.num_running == 0 and self.num_prefilling == 0

    # ── paged step planning ─────────────────────────────────────────────────

    def _alloc_device(self, dev: torch.device) -> None:
        B = self.max_batch_size
        max_tokens = B + self.chunked_prefill_size
        # decode takes at most one page per request; the chunks at most the
        # budget's pages plus one partial page per chunk
        self._max_new_pages = 2 * B + -(-self.chunked_prefill_size // KV_PAGE_SIZE) + 1
        upload_ints = B * _ENTRY_INTS + self._max_new_pages
        i32 = dict(dtype=torch.int32, device=dev)
        i64 = dict(dtype=torch.int64, device=dev)
        self._dev = dict(
            tables=torch.zeros(B, self.width, **i32),
            upload=torch.empty(upload_ints, **i32),
            slots=torch.empty(max_tokens, **i64),
            positions=torch.empty(max_tokens, **i64),
            cu=torch.zeros(B + 1, **i64),
            step_tables=torch.zeros(B, self.width, **i32),
            step_lens=torch.zeros(B, **i32),
            rows=torch.zeros(B, **i32),
            errors=_lib.DeviceErrors(dev),
        )
        self._pinned = [torch.empty(upload_ints, dtype=torch.int32, pin_memory=True)
                        for _ in range(self._RING)]
        self._events = [None] * self._RING
        self._ring = 0
        if self.block_manager is not None:
            # one block-manager round per step: per-id hash offsets and
            # lengths, the ops; read back: status and hits of the 2B ids,
            # the admits' (at most B) page rows
            W = self.block_manager.tables.shape[1]
            self._bm = dict(
                side=torch.cuda.Stream(dev),  # default priority, like every stream here
                meta_h=torch.empty(8 * (B + 1), dtype=torch.int64, pin_memory=True),
                meta_d=torch.empty(8 * (B + 1), **i64),
                # the results after each half of the round (a different buffer
                # each, so a late copy never overwrites what the host reads)
                back_a=torch.empty(B * (4 + W), dtype=torch.int32, pin_memory=True),
                back_b=torch.empty(B * (4 + W), dtype=torch.int32, pin_memory=True),
                count_h=torch.empty(2, dtype=torch.int64, pin_memory=True),
                errors=_lib.DeviceErrors(dev),
                uploaded=None,  # the previous round's upload (it reads meta_h)
            )

    def _retire(self, lst: list[InferenceRequest],
                ops: list[int] | None = None) -> list[InferenceRequest]:
        keep = []
        for r in lst:
            if r.is_done:
                if r.seq is not None and ops is not None:
                    # prefix reuse: the shareable pages go back through the
                    # block manager (to its LRU when cached), the rest to the
                    # private list
                    if r.fb > 0:
                        ops.append(-(r.bm_id + 1))
                        self._bm_ids.append(r.bm_id)
                        self.bm_held -= r.fb
                    self.kv_cache.free_pages(r.seq.page_table[r.fb:])
                    r.seq.page_table = []
                elif r.seq is not None:
                    self.kv_cache.free_pages(r.seq.page_table)
                    r.seq.page_table = []
                if r.row >= 0:
                    heapq.heappush(self._free_rows, r.row)
                    r.row = -1
            else:
                keep.append(r)
        return keep

    def plan_host(self) -> StepPlan | None:
        """The host half of ``plan_step``: scheduling decisions, page
        allocation and the upload record (``plan.upload``); device tensors are
        left unset. Returns None when nothing is scheduled."""
        if self.kv_cache is None:
            raise RuntimeError("plan_step needs a PagedKVCache (kv_cache=...)")
        if self._last is not None:
            raise RuntimeError("complete_step the previous plan before planning another")
        if self.block_manager is not None:
            return self._plan_host_prefix()
        cache = self.kv_cache
        P = KV_PAGE_SIZE
        with self.lock:
            self.running_batch = self._retire(self.running_batch)
            self.prefilling = self._retire(self.prefilling)
            rec = []  # (request, start, count, held, new)
            need_decode = 0
            for r in self.running_batch:
                seq = r.seq
                start = seq.seq_len
                held = len(seq.page_table)
                new = (start + P) // P - held   # pages to cover start + 1 tokens
                rec.append((r, start, 1, held, new))
                need_decode += new
            free = cache.num_free_pages - need_decode
            if free < 0:
                cache.alloc_pages(need_decode)  # raises the reference's OOM error
            budget = self.chunked_prefill_size
            prefill: list[tuple[InferenceRequest, int, int]] = []

            def take(r: InferenceRequest) -> int:
                nonlocal free, budget
                start = r.seq.seq_len
                held = len(r.seq.page_table)
                room = held * P - start + free * P
                n = min(len(r.input_ids) - r.num_prefilled, budget, room)
                if n <= 0:
                    return 0
                new = -(-(start + n) // P) - held
                free -= new
                budget -= n
                rec.append((r, start, n, held, new))
                prefill.append((r, start, n))
                return n

            stopped = False
            for r in self.prefilling:
                if budget == 0:
                    break
                if take(r) == 0:
                    stopped = True
                    break
            admitted = []
            while (not stopped and budget > 0 and self.waiting_queue
                   and len(self.running_batch) + len(self.prefilling) < self.max_batch_size):
                r = self.waiting_queue[0]
                if r.seq is None:
                    r.seq = SequenceKVState(max_pages=self.width)
                if take(r) == 0:
                    break
                self.waiting_queue.popleft()
                r.state = RequestState.PREFILLING
                r.row = heapq.heappop(self._free_rows)
                self.prefilling.append(r)
                admitted.append(r)
            if not rec:
                return None

            total_new = sum(e[4] for e in rec)
            pages = cache.alloc_pages(total_new)[::-1] if total_new else []
            n = len(rec)
            flat = []
            page_off = tok_off = 0
            for r, start, count, held, new in rec:
                flat += (r.row, start, count, held, new, page_off, tok_off, 0)
                if new:
                    r.seq.page_table += pages[page_off:page_off + new]
                page_off += new
                tok_off += count
                r.seq.seq_len = start + count
            for r, _, count in prefill:
                r.num_prefilled += count
            up = np.array(flat + pages, dtype=np.int32)
            decode = [e[0] for e in rec[:len(self.running_batch)]]
            for r, *_ in rec:
                r.dev_held = len(r.seq.page_table)
            plan = StepPlan(decode=decode, prefill=prefill, num_tokens=tok_off, upload=up,
                            slot_mapping=None, positions=None, cu_seqlens=None,
                            block_tables=None, seq_lens=None, rows=None, admitted=admitted,
                            fresh=list(range(n - len(admitted), n)))
            self._last = plan
            return plan

    def _plan_host_prefix(self) -> StepPlan | None:
        """plan_host with prefix reuse (the module docstring; the policy of
        oracle.sched.PrefixSchedulerModel)."""
        cache = self.kv_cache
        P = KV_PAGE_SIZE
        with self.lock:
            self._hash_queued()
            ops: list[int] = []
            self.running_batch = self._retire(self.running_batch, ops)
            self.prefilling = self._retire(self.prefilling, ops)
            entries = []  # (request, start, count)
            for r in self.running_batch:
                seq = r.seq
                if seq.seq_len >= len(seq.page_table) * P:
                    seq.page_table += cache.alloc_pages(1)  # the reference's OOM error if none
                entries.append((r, seq.seq_len, 1))
                seq.seq_len += 1
            budget = self.chunked_prefill_size
            prefill: list[tuple[InferenceRequest, int, int]] = []

            def chunk(r: InferenceRequest) -> None:
                nonlocal budget
                n = min(len(r.input_ids) - r.num_prefilled, budget)
                if n <= 0:
                    return
                start = r.seq.seq_len
                entries.append((r, start, n))
                prefill.append((r, start, n))
                r.seq.seq_len += n
                r.num_prefilled += n
                budget -= n

            for r in self.prefilling:
                chunk(r)
            cands: list[InferenceRequest] = []
            wc = budget
            while (wc > 0 and self.waiting_queue and cache.num_free_pages > len(cands)
                   and len(self.running_batch) + len(self.prefilling) + len(cands)
                   < self.max_batch_size):
                r = self.waiting_queue.popleft()
                r.fb = (len(r.input_ids) - 1) // P
                last = self.bm_held + r.fb > self.block_manager.num_pages
                r.row = heapq.heappop(self._free_rows)
                cands.append(r)
                self.bm_held += r.fb
                wc -= len(r.input_ids)
                if last:
                    break
            result = self._bm_round(ops, cands)
            admitted, skipped = [], 0
            for r in cands:
                table, r.hits = [], 0
                if r.fb > 0:
                    status, r.hits, table = result[r.bm_id]
                    if status != 0:  # OOM: only the last candidate can get it
                        self._bm_ids.appendleft(r.bm_id)
                        r.bm_id = -1
                        self.bm_held -= r.fb
                        heapq.heappush(self._free_rows, r.row)
                        r.row = -1
                        r.fb = 0
                        self.waiting_queue.appendleft(r)
                        continue
                r.page_hashes = None  # admitted: the block manager holds what it needs
                r.seq = SequenceKVState(max_pages=self.width)
                r.seq.page_table = list(table) + cache.alloc_pages(1)
                r.seq.seq_len = r.num_prefilled = r.hits * P
                r.dev_held = 0
                skipped += r.hits * P
                r.state = RequestState.PREFILLING
                self.prefilling.append(r)
                admitted.append(r)
                chunk(r)
            self.prefix_skipped += skipped
            ops += [r.bm_id for r in cands if r.fb > 0]
            if not entries:  # (the round above issued the releases)
                return None
            flat, pages, fresh = [], [], []
            tok_off = 0
            for i, (r, start, count) in enumerate(entries):
                new = r.seq.page_table[r.dev_held:]
                if r.dev_held == 0:
                    fresh.append(i)
                flat += (r.row, start, count, r.dev_held, len(new), len(pages), tok_off, 0)
                pages += new
                r.dev_held = len(r.seq.page_table)
                tok_off += count
            up = np.array(flat + pages, dtype=np.int32)
            decode = [e[0] for e in entries[:len(self.running_batch)]]
            plan = StepPlan(decode=decode, prefill=prefill, num_tokens=tok_off, upload=up,
                            slot_mapping=None, positions=None, cu_seqlens=None,
                            block_tables=None, seq_lens=None, rows=None, admitted=admitted,
                            fresh=fresh, skipped_tokens=skipped, bm_ops=ops)
            self._last = plan
            return plan

    def _hash_queued(self) -> None:
        """Page hashes of the shareable pages of every request queued since
        the last step, in one launch on the side stream. A request waits in
        the queue for at least this step, so its chain of SHA-256 pages (one
        lane walks it) is not on the admission's path; the hashes stay on the
        device with the request until its admission."""
        todo, self._unhashed = self._unhashed, []
        todo = [r for r in todo if (len(r.input_ids) - 1) // KV_PAGE_SIZE > 0]
        if not todo:
            return
        P = KV_PAGE_SIZE
        fbs = np.array([(len(r.input_ids) - 1) // P for r in todo], dtype=np.int64)
        cu_t = np.concatenate([[0], np.cumsum(fbs * P)]).astype(np.int64)
        tok = np.empty(int(cu_t[-1]), dtype=np.int64)
        for i, r in enumerate(todo):
            tok[cu_t[i]:cu_t[i + 1]] = r.input_ids[:int(fbs[i]) * P]
        offs = np.concatenate([cu_t, cu_t // P])
        dev = self.kv_cache.device
        side = self._bm["side"]
        with torch.cuda.stream(side):
            tok_d = torch.from_numpy(tok).to(dev)
            offs_d = torch.from_numpy(offs).to(dev)
            out = torch.empty(int(cu_t[-1]) // P, dtype=torch.int64, device=dev)
            _lib.call("mkv_block_hash_sha256", tok_d.data_ptr(), offs_d.data_ptr(),
                      offs_d[len(todo) + 1:].data_ptr(), len(todo), 8, out.data_ptr(),
                      self._bm["errors"].ptr(), side.cuda_stream)
        for i, r in enumerate(todo):
            r.page_hashes = out[int(cu_t[i]) // P:int(cu_t[i + 1]) // P]

    def _bm_round(self, ops: list[int], cands: list[InferenceRequest]) -> dict:
        """The step's block-manager work on the side stream: one mkv_bm_step
        with the releases and the candidates' admits (block-manager ids taken
        here; the candidates' page hashes were computed when they were
        queued). Waits for it only when there are admits, and returns
        {id: (status, hits, pages)}."""
        admits = [r for r in cands if r.fb > 0]
        for r in admits:
            r.bm_id = self._bm_ids.popleft()
            self._bm_ntok[r.bm_id] = r.fb * KV_PAGE_SIZE
        ops = list(ops) + [r.bm_id for r in admits]
        if not ops:
            return {}
        if self._dev is None:
            raise RuntimeError("prefix reuse runs the block manager on a ROCm GPU")
        b = self._bm
        bm = self.block_manager
        B = 2 * self.max_batch_size  # block-manager ids
        if b["uploaded"] is not None:
            b["uploaded"].synchronize()  # the previous round's upload read the staging buffer
            b["uploaded"] = None
        n = len(admits)
        admits = sorted(admits, key=lambda r: r.bm_id)
        per_id = np.zeros(B, dtype=np.int64)
        for r in admits:
            per_id[r.bm_id] = r.fb
        # one upload: per-id hash offsets (B+1, int64; the admits' hashes are
        # concatenated in id order, so the offsets are a prefix sum), then as
        # int32: per-id token counts (B), the ops (candidate order), the
        # admits' ids
        b["meta_h"].numpy()[:B + 1] = np.concatenate([[0], np.cumsum(per_id)])
        m32 = b["meta_h"].view(torch.int32).numpy()
        o_ntok = 2 * (B + 1)
        o_ops = o_ntok + B
        o_rows = o_ops + len(ops)
        m32[o_ntok:o_ops] = self._bm_ntok
        m32[o_ops:o_rows] = ops
        m32[o_rows:o_rows + n] = [r.bm_id for r in admits]
        side = b["side"]
        with torch.cuda.stream(side):
            md32 = b["meta_d"].view(torch.int32)
            md32[:o_rows + n].copy_(b["meta_h"].view(torch.int32)[:o_rows + n], non_blocking=True)
            b["uploaded"] = torch.cuda.Event()
            b["uploaded"].record(side)
            hashes = (torch.cat([r.page_hashes for r in admits]) if n
                      else b["meta_d"][:1])  # (no admit reads a hash)
            args = (md32[o_ops:o_rows], hashes, b["meta_d"][:B + 1], md32[o_ntok:o_ops])
            if not n:
                bm.step(*args)
                return {}
            # the committed-admit count around the many-CU half, and the
            # results read back after it and again after the one-workgroup
            # kernels (which wait for 96 KiB of LDS on a CU); the first copy
            # is final when every admit was committed
            ids = md32[o_rows:o_rows + n]
            count = b["count_h"]
            count[0:1].copy_(bm.spec_done_word(), non_blocking=True)
            bm.step_begin(*args)
            count[1:2].copy_(bm.spec_done_word(), non_blocking=True)
            early = self._bm_read_back(b["back_a"], ids, B, side)
            bm.step_end()
            late = self._bm_read_back(b["back_b"], ids, B, side)
        early[2].synchronize()
        c = count.numpy()
        if c[1] - c[0] == n:
            self.bm_early_rounds += 1
            sh, rows, _ = early
        else:
            self.bm_late_rounds += 1
            sh, rows, ev = late
            ev.synchronize()
        st_hits = sh.numpy().reshape(2, B)
        tables = rows.numpy().reshape(n, -1)
        return {r.bm_id: (int(st_hits[0, r.bm_id]), int(st_hits[1, r.bm_id]),
                          tables[i, :r.fb].tolist())
                for i, r in enumerate(admits)}

    def _bm_read_back(self, buf: torch.Tensor, ids: torch.Tensor, B: int,
                      stream: torch.cuda.Stream) -> tuple:
        """Copies (on ``stream``, the current one) the status and hits of every
        block-manager id and the table rows of ``ids`` into the pinned ``buf``;
        returns the two host views and an event after the copies."""
        bm = self.block_manager
        tab = bm.tables.index_select(0, ids)
        sh = buf[:2 * B]
        sh.copy_(bm.status_hits.view(-1), non_blocking=True)
        rows = buf[2 * B:2 * B + tab.numel()]
        rows.copy_(tab.view(-1), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        return sh, rows, ev

    def plan_step(self) -> StepPlan | None:
        """Schedules one step and writes its device tensors (one upload, one
        launch, on the current stream of the cache's device)."""
        if self.kv_cache is not None and self._dev is None:
            raise RuntimeError(
                f"plan_step runs its kernel on a ROCm GPU; the cache is on {self.kv_cache.device}")
        plan = self.plan_host()
        if plan is None:
            return None
        return self.launch_plan(plan)

    def launch_plan(self, plan: StepPlan) -> StepPlan:
        """The device half of ``plan_step``: uploads ``plan.upload`` and runs
        mkv_step_plan, filling the plan's device tensors."""
        if self._dev is None:
            raise RuntimeError("launch_plan needs the scheduler's pool on a ROCm GPU")
        if plan is not self._last or plan.slot_mapping is not None:
            raise RuntimeError("launch_plan takes the plan plan_host just returned, once")
        d = self._dev
        dev = self.kv_cache.device
        up = plan.upload
        n = plan.num_entries
        i = self._ring
        self._ring = (i + 1) % self._RING
        if self._events[i] is not None:
            self._events[i].synchronize()
        staging = self._pinned[i]
        staging.numpy()[:up.size] = up
        d["upload"][:up.size].copy_(staging[:up.size], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dev))
        self._events[i] = ev
        # per-step table width: the longest entry's pages (16-entry granules)
        npages = plan.upload[:n * _ENTRY_INTS].reshape(n, _ENTRY_INTS)
        width = int((npages[:, 3] + npages[:, 4]).max())
        width = min(self.width, -(-width // 16) * 16)
        base = d["upload"].data_ptr()
        _lib.call("mkv_step_plan", d["tables"].data_ptr(), d["tables"].stride(0), self.width,
                  self.max_batch_size, base, n, base + 4 * n * _ENTRY_INTS,
                  up.size - n * _ENTRY_INTS, self.kv_cache.num_pages, d["slots"].data_ptr(),
                  d["positions"].data_ptr(), plan.num_tokens, d["step_tables"].data_ptr(),
                  d["step_tables"].stride(0), width, d["step_lens"].data_ptr(),
                  d["rows"].data_ptr(), d["cu"].data_ptr(), d["errors"].ptr(),
                  _lib.stream_of(dev))
        T = plan.num_tokens
        plan.slot_mapping = d["slots"][:T]
        plan.positions = d["positions"][:T]
        plan.cu_seqlens = d["cu"][:n + 1]
        plan.block_tables = d["step_tables"][:n, :width]
        plan.seq_lens = d["step_lens"][:n]
        plan.rows = d["rows"][:n]
        if self.state_pool is not None and plan.fresh:
            # requests whose first entry this is start from zero GDN states
            idx = plan.fresh
            if idx == list(range(idx[0], idx[0] + len(idx))):
                self.state_pool.reset(plan.rows[idx[0]:idx[0] + len(idx)])
            else:
                self.state_pool.reset(plan.rows[torch.tensor(idx, device=plan.rows.device)])
        return plan

    def complete_step(self, plan: StepPlan, next_tokens=None) -> list[InferenceRequest]:
        """Applies one sampled token per entry (decode entries, then chunks;
        a chunk that did not finish its prompt ignores its token). Returns the
        requests that finished."""
        if plan is not self._last:
            raise RuntimeError("complete_step takes the last plan, once")
        self._last = None
        toks = [0] * plan.num_entries if next_tokens is None else list(next_tokens)
        if len(toks) != plan.num_entries:
            raise ValueError(f"{len(toks)} tokens for {plan.num_entries} entries")
        done = []
        now = time.time()
        eos, max_len = self.eos_token_id, self.max_seq_len
        nd = len(plan.decode)
        with self.lock:
            for i, r in enumerate(plan.decode + [r for r, _, _ in plan.prefill]):
                if i >= nd:
                    if r.num_prefilled < len(r.input_ids):
                        continue
                    r.state = RequestState.DECODING
                    r.first_token_at = now
                    self.prefilling.remove(r)
                    self.running_batch.append(r)
                tok = int(toks[i])
                gen = r.generated_tokens
                gen.append(tok)
                if (len(gen) >= r.max_new_tokens or tok == eos or r.seq.seq_len >= max_len):
                    r.state = RequestState.FINISHED
                    r.finished_at = now
                    done.append(r)
        return done

    def check_errors(self) -> None:
        """Synchronises and raises MkvDeviceError if a step plan was malformed
        (or, with prefix reuse, a block-manager round flagged a fault)."""
        if self._dev is not None:
            self._dev["errors"].check("ContinuousBatchScheduler")
        if self.block_manager is not None and self._dev is not None:
            self._bm["side"].synchronize()
            self._bm["errors"].check("ContinuousBatchScheduler page hashes")
            self.block_manager.check_errors()
