"""Continuous-batching scheduler with chunked prefill, on the CPU (oracle; test
infrastructure only).

``ReferenceScheduler`` restates ``ContinuousBatchScheduler`` of
muserve/scheduler.py:54-123: a FIFO waiting queue, a running batch, and a
step that decodes every running request and admits waiting requests while
running + admitted < max_batch_size.

``ChunkedSchedulerModel`` is the paged step the library drives from that
scheduler. The reference has no chunked prefill in its scheduler, only the
chunk size muserve/config.py:40; the policy below is the library's and is
stated once here, token by token:

1. Retire: FINISHED requests leave the running batch (its order), then the
   prefilling list (its order); each frees its pages
   (``PoolModel.release(page_table)``, muserve/kv_cache.py:88-91) and its
   batch row.
2. Decode: every running request adds one token (``SeqModel.add_tokens``,
   the per-token ``alloc_pages(1)`` loop of muserve/scripts/test_kv_cache.py:88-92);
   an empty pool raises the reference's OOM error.
3. Prefill, with a budget of ``chunk`` tokens per step: first the requests
   already prefilling (admission order), then waiting requests admitted in
   FIFO order while running + prefilling < max_batch_size
   (muserve/scheduler.py:86-96). A request adds prompt tokens one at a time
   while it has prompt left, budget left, and a page for the token (its last
   page has room, or the pool is not empty). The first request that gets no
   token ends the prefill for this step (a waiting one stays queued). An
   admitted request takes the smallest free row.
4. The step's entries are the decode tokens (running order), then the prefill
   chunks (prefilling order); every token's slot is page*16 + position%16 of
   its sequence's page table after the step.
5. ``complete(tokens)``: a decode entry appends its sampled token; a chunk
   that completed its prompt appends its first token, becomes DECODING and
   joins the running batch (``finish_prefill``, muserve/scheduler.py:100-106).
   A request finishes when it has max_new_tokens tokens, samples eos, or its
   next decode would pass max_seq_len (``finish_request``, :108-111).
"""
from __future__ import annotations

from collections import deque

import numpy as np

from oracle.paged import PAGE, PoolModel, SeqModel

WAITING, PREFILLING, DECODING, FINISHED = "waiting", "prefilling", "decoding", "finished"


class Req:
    def __init__(self, rid, prompt_len: int, max_new_tokens: int = 256):
        self.rid = rid
        self.prompt_len = prompt_len
        self.max_new_tokens = max_new_tokens
        self.state = WAITING
        self.generated: list[int] = []
        self.seq = SeqModel()
        self.row = -1
        self.prefilled = 0


class ReferenceScheduler:
    """muserve/scheduler.py:54-123 without the lock and timestamps."""

    def __init__(self, max_batch_size: int = 8):
        self.max_batch_size = max_batch_size
        self.waiting: deque = deque()
        self.running: list = []

    def add_request(self, req) -> None:                      # :69-71
        self.waiting.append(req)

    def schedule_step(self):                                  # :73-98
        self.running = [r for r in self.running if r.state != FINISHED]
        decode = list(self.running)
        prefill = []
        while self.waiting and len(self.running) + len(prefill) < self.max_batch_size:
            req = self.waiting.popleft()
            req.state = PREFILLING
            prefill.append(req)
        return prefill, decode

    def finish_prefill(self, reqs) -> None:                   # :100-106
        for r in reqs:
            r.state = DECODING
            self.running.append(r)

    def finish_request(self, req) -> None:                    # :108-111
        req.state = FINISHED


class ChunkedSchedulerModel:
    def __init__(self, max_batch_size: int, chunk: int, pool: PoolModel, max_seq_len: int,
                 eos: int | None = None):
        self.max_batch_size = max_batch_size
        self.chunk = chunk
        self.pool = pool
        self.max_seq_len = max_seq_len
        self.width = -(-max_seq_len // PAGE)
        self.eos = eos
        self.waiting: deque = deque()
        self.running: list = []
        self.prefilling: list = []
        self.rows_in_use: set[int] = set()
        self.last: list | None = None  # the last step's entries: (req, kind, start, count)

    def add(self, req: Req) -> None:
        self.waiting.append(req)

    def _free_row(self) -> int:
        r = 0
        while r in self.rows_in_use:
            r += 1
        self.rows_in_use.add(r)
        return r

    def _retire(self, lst: list) -> list:
        keep = []
        for r in lst:
            if r.state == FINISHED:
                self.pool.release(r.seq.page_table)
                r.seq.page_table = []
                self.rows_in_use.discard(r.row)
                r.row = -1
            else:
                keep.append(r)
        return keep

    def _take(self, r: Req, budget: int) -> int:
        """Adds prompt tokens one at a time; returns how many it added."""
        n = 0
        while r.prefilled + n < r.prompt_len and n < budget:
            if r.seq.needs_new_page() and self.pool.num_free == 0:
                break
            n += 1
            r.seq.add_tokens(self.pool, 1)
        return n

    def step(self) -> dict:
        self.running = self._retire(self.running)
        self.prefilling = self._retire(self.prefilling)
        entries, slots, positions = [], [], []
        for r in self.running:
            start = r.seq.seq_len
            slots += r.seq.add_tokens(self.pool, 1)
            positions.append(start)
            entries.append((r, "decode", start, 1))
        budget = self.chunk
        stopped = False
        for r in self.prefilling:
            if budget == 0:
                break
            start = r.seq.seq_len
            n = self._take(r, budget)
            if n == 0:
                stopped = True
                break
            self._record(r, start, n, slots, positions, entries)
            budget -= n
        while (not stopped and budget > 0 and self.waiting
               and len(self.running) + len(self.prefilling) < self.max_batch_size):
            r = self.waiting[0]
            start = r.seq.seq_len
            n = self._take(r, budget)
            if n == 0:
                break
            self.waiting.popleft()
            r.state = PREFILLING
            r.row = self._free_row()
            self.prefilling.append(r)
            self._record(r, start, n, slots, positions, entries)
            budget -= n
        self.last = entries
        cu = [0]
        for e in entries:
            cu.append(cu[-1] + e[3])
        return {
            "rids": [e[0].rid for e in entries],
            "kinds": [e[1] for e in entries],
            "starts": [e[2] for e in entries],
            "counts": [e[3] for e in entries],
            "rows": [e[0].row for e in entries],
            "slots": slots,
            "positions": positions,
            "cu_seqlens": cu,
            "lens": [e[0].seq.seq_len for e in entries],
            # page_table_tensor of every entry (muserve/kv_cache.py:149-158)
            "tables": [list(e[0].seq.page_table) + [0] * (self.width - len(e[0].seq.page_table))
                       for e in entries],
        }

    def _record(self, r, start, n, slots, positions, entries) -> None:
        r.prefilled += n
        pos = range(start, start + n)
        slots += [r.seq.page_table[p // PAGE] * PAGE + p % PAGE for p in pos]
        positions += list(pos)
        entries.append((r, "prefill", start, n))

    def complete(self, tokens: list[int] | None = None) -> list:
        """Applies the sampled tokens of the last step; returns the requests
        that finished."""
        done = []
        for i, (r, kind, start, n) in enumerate(self.last or []):
            tok = 0 if tokens is None else tokens[i]
            if kind == "prefill":
                if r.prefilled < r.prompt_len:
                    continue
                r.state = DECODING
                self.prefilling.remove(r)
                self.running.append(r)
            r.generated.append(tok)
            if (len(r.generated) >= r.max_new_tokens or (self.eos is not None and tok == self.eos)
                    or r.seq.seq_len >= self.max_seq_len):
                r.state = FINISHED
                done.append(r)
        self.last = None
        return done


class PReq(Req):
    """A request with its prompt's token ids (prefix reuse needs them)."""

    def __init__(self, rid, tokens, max_new_tokens: int = 256):
        super().__init__(rid, len(tokens), max_new_tokens)
        self.tokens = list(tokens)
        self.fb = (len(tokens) - 1) // PAGE  # shareable pages: full pages before the last token
        self.hits = 0
        self.bm_id = -1


class PrefixSchedulerModel(ChunkedSchedulerModel):
    """``ChunkedSchedulerModel`` with prefix reuse through the block manager
    (``oracle.blocks.BlockManagerModel``). The pool is split: the block
    manager owns its pages (the cacheable prompt pages), a LIFO list
    (``PoolModel``) the rest (each request's private pages). The policy, in
    the order a step applies it:

    1. Retire as before; a finished request also releases its block-manager
       pages (``release(row)``, in retire order) and returns its private pages
       to the list.
    2. Decode as before (new pages from the private list).
    3. Prefill the prefilling requests (admission order) with the budget.
       Every prompt page was taken at admission. A hit page is never read
       before it is written: the request that took it fresh was admitted
       earlier, so it comes earlier in this order, and the budget only
       reaches a later request once every earlier one has its whole prompt
       (the chunk of a request is its remaining prompt or the remaining
       budget). ``_chunk`` asserts it.
    4. Admission: while the budget assumed for the candidates so far (their
       whole prompts, as if nothing were cached) leaves some budget, a row is
       free and the private list has a page for every candidate, the head of
       the queue becomes a candidate and takes the smallest free row. Its
       shareable pages are fb = (n - 1) // 16, the full pages before its last
       prompt token. A candidate whose fb would push the sum of fb over
       admitted requests past the block manager's pages is the last candidate
       of the step (the block manager decides it exactly).
    5. The block manager runs the step's releases, then the candidates' admits
       (``admit(id, page hashes of the first fb pages, 16 fb)``; none when
       fb is 0). Its request ids come from a FIFO of 2 x max_batch_size ids:
       an admit takes the front id, a release puts its id at the back, so an
       id released in a step is not taken again in that step. An OOM
       candidate goes back to the head of the queue, its id back to the front
       of the FIFO, and frees its row. An admitted one takes its tail page from the private list
       (the page of its last prompt token, where its decode continues), starts
       with its k hit pages' 16 k tokens in the cache (skipped), and takes a
       chunk from the budget.
    6. Entries, slots and ``complete`` as in ``ChunkedSchedulerModel``.
    """

    def __init__(self, max_batch_size: int, chunk: int, bm, private: PoolModel, max_seq_len: int,
                 eos: int | None = None):
        super().__init__(max_batch_size, chunk, private, max_seq_len, eos)
        self.bm = bm
        self.bm_held = 0  # sum of fb over requests admitted to the block manager
        self.writer: dict[int, tuple] = {}  # page -> (request, table index) not yet written
        self.skipped = 0
        self.bm_ids = deque(range(2 * max_batch_size))

    def _unwritten_hits(self, r: PReq) -> list[int]:
        """r's hit pages whose writer has not yet written them."""
        out = []
        for j in range(r.hits):
            w = self.writer.get(r.seq.page_table[j])
            if w is not None and w[0].prefilled < (w[1] + 1) * PAGE:
                out.append(r.seq.page_table[j])
        return out

    def _chunk(self, r: PReq, budget: int, slots, positions, entries) -> int:
        if budget == 0:
            return 0
        assert not self._unwritten_hits(r), "a hit page would be read before it is written"
        n = min(r.prompt_len - r.prefilled, budget)
        start = r.seq.seq_len
        r.seq.seq_len += n
        self._record(r, start, n, slots, positions, entries)
        return n

    def step(self) -> dict:
        from oracle.sha import page_hashes
        ops = []

        def retire(lst):
            keep = []
            for r in lst:
                if r.state == FINISHED:
                    if r.fb > 0:
                        ops.append(-(r.bm_id + 1))
                        self.bm.release(r.bm_id)
                        self.bm_ids.append(r.bm_id)
                        self.bm_held -= r.fb
                    self.pool.release(r.seq.page_table[r.fb:])
                    r.seq.page_table = []
                    self.rows_in_use.discard(r.row)
                    r.row = -1
                else:
                    keep.append(r)
            return keep

        self.running = retire(self.running)
        self.prefilling = retire(self.prefilling)
        entries, slots, positions = [], [], []
        for r in self.running:
            start = r.seq.seq_len
            slots += r.seq.add_tokens(self.pool, 1)
            positions.append(start)
            entries.append((r, "decode", start, 1))
        budget = self.chunk
        for r in self.prefilling:
            budget -= self._chunk(r, budget, slots, positions, entries)
        cands = []
        wc = budget
        while (wc > 0 and self.waiting and self.pool.num_free > len(cands)
               and len(self.running) + len(self.prefilling) + len(cands) < self.max_batch_size):
            r = self.waiting.popleft()
            last = self.bm_held + r.fb > self.bm.P
            r.row = self._free_row()
            cands.append(r)
            self.bm_held += r.fb
            wc -= r.prompt_len
            if last:
                break
        admitted, skipped = [], 0
        for r in cands:
            table = []
            if r.fb > 0:
                r.bm_id = self.bm_ids.popleft()
                ops.append(r.bm_id)
                res = self.bm.admit(r.bm_id, page_hashes(np.asarray(r.tokens[:r.fb * PAGE],
                                                                    dtype=np.int64)), r.fb * PAGE)
                if res["status"] != 0:  # OOM: only the last candidate can get it
                    self.bm_ids.appendleft(r.bm_id)
                    r.bm_id = -1
                    self.bm_held -= r.fb
                    self.rows_in_use.discard(r.row)
                    r.row = -1
                    self.waiting.appendleft(r)
                    continue
                table, r.hits = res["table"], res["hits"]
            r.seq.page_table = list(table) + self.pool.alloc(1)
            r.seq.seq_len = r.prefilled = r.hits * PAGE
            skipped += r.hits * PAGE
            for j in range(r.hits, r.fb):
                self.writer[table[j]] = (r, j)
            r.state = PREFILLING
            self.prefilling.append(r)
            admitted.append(r)
            budget -= self._chunk(r, budget, slots, positions, entries)
        self.writer = {p: w for p, w in self.writer.items() if w[0].prefilled < (w[1] + 1) * PAGE}
        self.skipped += skipped
        self.last = entries
        cu = [0]
        for e in entries:
            cu.append(cu[-1] + e[3])
        return {
            "rids": [e[0].rid for e in entries],
            "kinds": [e[1] for e in entries],
            "starts": [e[2] for e in entries],
            "counts": [e[3] for e in entries],
            "rows": [e[0].row for e in entries],
            "slots": slots,
            "positions": positions,
            "cu_seqlens": cu,
            "lens": [e[0].seq.seq_len for e in entries],
            "tables": [list(e[0].seq.page_table) + [0] * (self.width - len(e[0].seq.page_table))
                       for e in entries],
            "ops": ops,
            "admitted": [(r.rid, r.row, r.hits) for r in admitted],
            "skipped": skipped,
        }
