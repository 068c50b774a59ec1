"""GPU-resident block manager for prefix caching (refcounts, copy-on-write,
LRU eviction), driving mkv_bm_step.

The reference caches whole prefixes in an OrderedDict
(muserve/model/prefix_cache.py:46-105) and hands out pages from a LIFO list
(muserve/kv_cache.py:77-91). ``BlockManager`` does both at page granularity
on the device: a request's full 16-token pages are keyed by the SHA-256 prefix
hash of ``PrefixCache._hash_tokens`` (``prefix_hash.page_hashes``), the
longest run of leading cached pages is shared (refcounted), the rest come from
the free stack or by evicting the least recently released cached page, and a
forked request's partial last page is copied on write. A step's admits are
resolved together on many CUs against the state at their start, every
prediction checked; from the first admit that could differ from the
sequential order, one workgroup resolves the rest in op order (admits eight
at a time). A step of at most 8 ops runs on one workgroup, one op at a time.
Eviction order is deterministic and equal to the sequential OrderedDict
model. Page hashes must be prefix keys (a hash at position i equal in two
requests only if their hashes at every earlier position are).

Typical step for a batch of requests (all on the stream, no host sync)::

    hashes, cu_pages = prefix_hash.page_hashes(tokens, cu_tokens)
    bm.step(ops, hashes, cu_pages_dev, num_tokens_dev)
    bm.copy_on_write(cache, first_request, last_request)
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from muserve_amd import _lib

STATUS_ADMITTED, STATUS_OOM, STATUS_BAD, STATUS_RELEASED = 0, 1, 2, 3
_FREE_TOP, _HEAD, _TAIL, _NEXT_STAMP, _EVICTABLE, _TOMBS, _LOG_LEN, _SPEC_DONE, _SPEC_LEFT = range(9)


def admit_op(r: int) -> int:
    return r


def release_op(r: int) -> int:
    return -(r + 1)


class BlockManager:
    def __init__(self, num_pages: int, max_requests: int, max_pages_per_request: int,
                 device: torch.device | str = "cuda", free_order=None,
                 evict_log_capacity: int = 0):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("BlockManager runs on a ROCm GPU only")
        self.num_pages = num_pages
        lib = _lib.load()
        nbytes = lib.mkv_bm_state_bytes(num_pages)
        if nbytes <= 0:
            raise ValueError(f"bad page count {num_pages}")
        lay = (ctypes.c_int64 * 10)()
        _lib.call("mkv_bm_layout", num_pages, ctypes.addressof(lay))
        # table capacity, ring capacity, byte offsets of counters, table, page
        # records, free stack, ring, last-occurrence slots, release-run
        # scratch; total bytes
        self.layout = dict(zip(("C", "Q", "ctr", "ent", "rec", "free", "ring", "last", "run",
                                "bytes"), lay))
        self.state = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        if self.state.data_ptr() % 256:
            raise RuntimeError("state buffer is not 256-byte aligned")
        order = None
        if free_order is not None:
            order = torch.as_tensor(np.asarray(free_order, dtype=np.int32)).to(self.device)
            if order.numel() != num_pages:
                raise ValueError("free_order must list every page once")
        stream = _lib.stream_of(self.device)
        _lib.call("mkv_bm_init", self.state.data_ptr(), num_pages, _lib.ptr(order), stream)
        R, W = max_requests, max_pages_per_request
        i32 = dict(dtype=torch.int32, device=self.device)
        self.tables = torch.full((R, W), -1, **i32)
        # per request id: status and leading hits, the two rows of one tensor
        # (a caller reads both back with one copy)
        self.status_hits = torch.full((2, R), -1, **i32)
        self.status, self.hits = self.status_hits[0], self.status_hits[1]
        self.child_last = torch.full((R,), -1, **i32)
        self.cow_src = torch.full((R,), -1, **i32)
        self.cow_dst = torch.full((R,), -1, **i32)
        self.evict_log = torch.full((max(evict_log_capacity, 1),), -1, **i32)
        self.evict_log_capacity = evict_log_capacity
        self.errors = _lib.DeviceErrors(self.device)
        self._pending = None  # step_begin's arguments until step_end
        self._keep = None

    def step(self, ops: torch.Tensor, page_hashes: torch.Tensor, hash_offsets: torch.Tensor,
             num_tokens: torch.Tensor) -> None:
        """Runs ops (int32: r admits request r, -(r+1) releases it) in order.
        page_hashes: int64 device tensor of u64 page-hash bit patterns;
        hash_offsets: int64 [max_requests+1] offsets into it per request id;
        num_tokens: int32 [max_requests] prompt lengths."""
        if self._pending is not None:
            raise RuntimeError("step while a step_begin awaits its step_end")
        args, keep = self._step_args(ops, page_hashes, hash_offsets, num_tokens)
        _lib.call("mkv_bm_step", *args)
        self._keep = keep  # the launches read these buffers: keep them until the next step

    def step_begin(self, ops: torch.Tensor, page_hashes: torch.Tensor, hash_offsets: torch.Tensor,
                   num_tokens: torch.Tensor) -> None:
        """The first half of ``step`` (same arguments): the release run and the
        many-CU resolution of the admits after it. ``step_end`` must follow, on
        the same stream, before anything else uses the manager. In between, the
        admits the resolution committed (the growth of ``spec_done_word``) have
        their final status, hits and table rows: when that growth equals the
        number of admits in ops, ``step_end`` has nothing left to run."""
        if self._pending is not None:
            raise RuntimeError("step_begin twice without step_end")
        args, keep = self._step_args(ops, page_hashes, hash_offsets, num_tokens)
        _lib.call("mkv_bm_step_begin", *args)
        # the pending step's tensors stay with it: step_end's launches read them
        self._pending = (args, keep)

    def step_end(self) -> None:
        """The second half of ``step``: the one-workgroup tail kernel over the
        ops the resolution left."""
        if self._pending is None:
            raise RuntimeError("step_end without step_begin")
        (args, keep), self._pending = self._pending, None
        _lib.call("mkv_bm_step_end", *args)
        self._keep = keep  # until the next step: the launches may still be running

    def spec_done_word(self) -> torch.Tensor:
        """Device view (int64, one element) of the running count of admits the
        many-CU resolution committed, for an asynchronous copy."""
        return self._arr("ctr", 16, torch.int64)[_SPEC_DONE:_SPEC_DONE + 1]

    def _step_args(self, ops, page_hashes, hash_offsets, num_tokens) -> tuple:
        if not (isinstance(ops, torch.Tensor) and ops.device.type == "cuda"):
            host = np.asarray(ops.cpu() if isinstance(ops, torch.Tensor) else ops, dtype=np.int64)
            req = np.where(host >= 0, host, -(host + 1))
            if host.size and (req.max() >= self.tables.shape[0]):
                raise IndexError(f"op names request {int(req.max())} >= {self.tables.shape[0]}")
            ops = torch.from_numpy(host.astype(np.int32))
        if hash_offsets.numel() != self.tables.shape[0] + 1 or num_tokens.numel() != self.tables.shape[0]:
            raise ValueError("hash_offsets needs max_requests+1 entries and num_tokens max_requests")
        ops = ops.to(device=self.device, dtype=torch.int32).contiguous()
        hash_offsets = hash_offsets.to(device=self.device, dtype=torch.int64).contiguous()
        num_tokens = num_tokens.to(device=self.device, dtype=torch.int32).contiguous()
        page_hashes = page_hashes.to(device=self.device).contiguous()
        if page_hashes.dtype != torch.int64:
            raise TypeError("page_hashes must hold u64 bit patterns in an int64 tensor")
        _lib.require_gpu(ops, hash_offsets, num_tokens, self.state)
        # the tensors the launches read go back with the arguments: the caller
        # keeps them alive until the launches are ordered before any reuse
        keep = (ops, page_hashes, hash_offsets, num_tokens)
        return (self.state.data_ptr(), self.num_pages, ops.data_ptr(),
                ops.numel(), self.tables.shape[0], page_hashes.data_ptr(), hash_offsets.data_ptr(),
                num_tokens.data_ptr(), self.tables.data_ptr(), self.tables.stride(0),
                self.tables.shape[1], self.hits.data_ptr(), self.child_last.data_ptr(),
                self.cow_src.data_ptr(), self.cow_dst.data_ptr(), self.status.data_ptr(),
                self.evict_log.data_ptr(), self.evict_log_capacity, self.errors.ptr(),
                _lib.stream_of(self.device)), keep

    def probe(self, page_hashes: torch.Tensor, hash_offsets: torch.Tensor
              ) -> tuple[torch.Tensor, torch.Tensor]:
        """Read-only lookup (no LRU touch, no pin) of the page hashes of
        len(hash_offsets)-1 requests: (page id per hash or -1, leading hits per
        request). Ordered after earlier steps on the same stream."""
        hash_offsets = hash_offsets.to(device=self.device, dtype=torch.int64).contiguous()
        page_hashes = page_hashes.to(device=self.device).contiguous()
        if page_hashes.dtype != torch.int64:
            raise TypeError("page_hashes must hold u64 bit patterns in an int64 tensor")
        n = hash_offsets.numel() - 1
        pages = torch.empty(page_hashes.numel(), dtype=torch.int32, device=self.device)
        hits = torch.empty(max(n, 0), dtype=torch.int32, device=self.device)
        if n > 0:
            _lib.call("mkv_hash_probe", self.state.data_ptr(), self.num_pages,
                      page_hashes.data_ptr(), hash_offsets.data_ptr(), n, pages.data_ptr(),
                      hits.data_ptr(), self.errors.ptr(), _lib.stream_of(self.device))
        return pages, hits

    def copy_on_write(self, cache, first: int = 0, last: int | None = None) -> None:
        """Copies every admitted request's shared partial page to its child's
        private page (requests first..last-1; pairs without a copy are -1)."""
        cache.copy_pages(self.cow_src[first:last], self.cow_dst[first:last])

    def check_errors(self) -> None:
        self.errors.check("BlockManager")

    # -- inspection (synchronises) --
    def _arr(self, name: str, count: int, dtype: torch.dtype) -> torch.Tensor:
        off = self.layout[name]
        esz = torch.empty((), dtype=dtype).element_size()
        return self.state[off:off + count * esz].view(dtype)

    def counters(self) -> list[int]:
        return self._arr("ctr", 16, torch.int64).cpu().tolist()

    def snapshot(self) -> dict:
        """Host copy of the bookkeeping: free stack (bottom..top), live LRU
        order (oldest first), refcounts, cached flags, page hashes (u64)."""
        P, Q = self.num_pages, self.layout["Q"]
        ctr = self.counters()
        # page record: i32 ref, i32 flag, u32 stamp, i32 table slot, u64 hash, u64 unused
        rec = self._arr("rec", P * 8, torch.int32).cpu().numpy().reshape(P, 8)
        ref, flag = rec[:, 0], rec[:, 1]
        stamp = rec[:, 2].view(np.uint32)
        phash = rec.view(np.uint64).reshape(P, 4)[:, 2]
        free = self._arr("free", P, torch.int32).cpu().numpy()[:ctr[_FREE_TOP]]
        ring = self._arr("ring", Q, torch.int64).cpu().numpy().view(np.uint64)
        rpg = (ring & 0xFFFFFFFF).astype(np.int64)
        rst = (ring >> 32).astype(np.int64)
        lru = []
        for pos in range(ctr[_HEAD], ctr[_TAIL]):
            pg, st = int(rpg[pos % Q]), int(rst[pos % Q])
            if flag[pg] & 1 and ref[pg] == 0 and int(stamp[pg]) == st:
                lru.append(pg)
        cached = flag & 1
        # table entry: u64 key, i32 page, i32 copy of the page's refcount
        ent = self._arr("ent", self.layout["C"] * 4, torch.int32).cpu().numpy().reshape(-1, 4)
        cp = np.nonzero(cached)[0]
        slot = rec[cp, 3]
        table_ok = bool(np.all(ent[slot, 2] == cp) and np.all(ent[slot, 3] == ref[cp]) and
                        np.all(ent.view(np.uint64).reshape(-1, 2)[slot, 0] == phash[cp]) and
                        int(np.count_nonzero(ent[:, 2] >= 0)) == len(cp))
        tombs_ok = int(np.count_nonzero(ent[:, 2] == -2)) == ctr[_TOMBS]
        # the release-run scratch's last-occurrence slots are -1 between steps
        last_ok = bool(np.all(self._arr("last", P, torch.int32).cpu().numpy() == -1))
        return {"free": free.tolist(), "lru": lru, "ref": ref.tolist(), "table_ok": table_ok,
                "last_ok": last_ok, "tombs_ok": tombs_ok,
                "cached": cached.tolist(),
                "hash": [int(phash[p]) if cached[p] else None for p in range(P)],
                "evictable": ctr[_EVICTABLE], "log_len": ctr[_LOG_LEN],
                # admits resolved by the many-CU speculation / covered by it but
                # left to the sequential kernels, since the manager was made
                "spec_done": ctr[_SPEC_DONE], "spec_left": ctr[_SPEC_LEFT]}
