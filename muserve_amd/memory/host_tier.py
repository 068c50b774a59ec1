"""Host tier: prefix-cache state in pinned host memory.

The reference keeps prefix-cache entries in host RAM by ``tensor.cpu()``, a
synchronous copy into pageable memory, and brings them back with
``.to(device, non_blocking=True)``, which from pageable memory is not
asynchronous (muserve/model/prefix_cache.py:36-44). Here:

* ``PinnedArena``: one pinned allocation (torch ``pin_memory``, i.e.
  hipHostMalloc) carved into 256-byte-aligned ranges, first fit with
  coalescing on free.
* Dense tensors (the hidden state, per-layer GDN states) move by DMA
  (``copy_`` with ``non_blocking``, hipMemcpyAsync on pinned memory).
* Blocks of the library's pools (the KV pages of a prefix, fp8 scales, a GDN
  state slot across layers) move with ``mkv_pack_blocks`` /
  ``mkv_unpack_blocks``: the kernel reads the scattered blocks from HBM and
  writes the pinned arena across the host link itself, or the reverse, with no
  staging copy.
* All arena traffic runs on one copy stream per tier, a default-priority side
  stream. It waits for the caller's stream before reading device data, and the
  caller's stream waits for it before using restored data. Because the copy
  stream is the only user of the arena, a range freed by an eviction and
  reused is never written while an earlier restore still reads it.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

import torch

from muserve_amd import _lib

ALIGN = 256


class PinnedArena:
    """A pinned host buffer handing out aligned byte ranges (first fit)."""

    def __init__(self, nbytes: int, pinned: bool = True):
        if nbytes <= 0:
            raise ValueError("arena size must be positive")
        self.nbytes = int(nbytes)
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=pinned)
        self._free: list[tuple[int, int]] = [(0, self.nbytes)]  # (offset, length), by offset

    @staticmethod
    def rounded(n: int) -> int:
        return max(ALIGN, (int(n) + ALIGN - 1) // ALIGN * ALIGN)

    def alloc(self, n: int) -> int | None:
        """Offset of a free range of n bytes (rounded up to 256), or None."""
        n = self.rounded(n)
        for i, (off, ln) in enumerate(self._free):
            if ln >= n:
                if ln == n:
                    del self._free[i]
                else:
                    self._free[i] = (off + n, ln - n)
                return off
        return None

    def free(self, off: int, n: int) -> None:
        n = self.rounded(n)
        if off < 0 or off + n > self.nbytes:
            raise ValueError(f"range {off}+{n} outside the arena")
        lo, hi = 0, len(self._free)
        while lo < hi:  # insertion point by offset
            mid = (lo + hi) // 2
            if self._free[mid][0] < off:
                lo = mid + 1
            else:
                hi = mid
        if lo > 0 and self._free[lo - 1][0] + self._free[lo - 1][1] > off:
            raise ValueError(f"range {off}+{n} overlaps a free range (double free)")
        if lo < len(self._free) and off + n > self._free[lo][0]:
            raise ValueError(f"range {off}+{n} overlaps a free range (double free)")
        self._free.insert(lo, (off, n))
        if lo + 1 < len(self._free) and off + n == self._free[lo + 1][0]:  # merge right
            self._free[lo] = (off, n + self._free[lo + 1][1])
            del self._free[lo + 1]
        if lo > 0 and self._free[lo - 1][0] + self._free[lo - 1][1] == off:  # merge left
            self._free[lo - 1] = (self._free[lo - 1][0], self._free[lo - 1][1] + self._free[lo][1])
            del self._free[lo]

    def free_bytes(self) -> int:
        return sum(ln for _, ln in self._free)

    def largest_free(self) -> int:
        return max((ln for _, ln in self._free), default=0)

    def view(self, off: int, n: int) -> torch.Tensor:
        return self.buf[off:off + n]


@dataclass
class HostTensor:
    """A dense tensor held in the arena."""
    off: int
    nbytes: int
    shape: tuple
    dtype: torch.dtype

    def nelement(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def element_size(self) -> int:
        return torch.empty((), dtype=self.dtype).element_size()


@dataclass
class HostBlocks:
    """Blocks of a layered pool held in the arena, plane-major."""
    off: int
    nbytes: int
    planes: int
    n: int
    block_bytes: int


def pool_layout(pool: torch.Tensor, block_dims: int) -> tuple[int, int, int, int]:
    """(planes, plane_stride, block_bytes, pool_blocks) of a contiguous pool
    [planes..., blocks, block...] whose last ``block_dims`` dims form a block."""
    if not pool.is_contiguous():
        raise ValueError("pool must be contiguous")
    lead = pool.shape[:pool.dim() - block_dims]
    if len(lead) < 1:
        raise ValueError("pool needs a block dimension")
    blocks = lead[-1]
    planes = 1
    for d in lead[:-1]:
        planes *= d
    block_bytes = pool.element_size()
    for d in pool.shape[pool.dim() - block_dims:]:
        block_bytes *= d
    return planes, blocks * block_bytes, block_bytes, blocks


class HostTier:
    """Pinned arena plus the copy stream that moves data in and out of it."""

    def __init__(self, nbytes: int, device: torch.device | str = "cuda"):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("the host tier moves device data: it needs a ROCm GPU")
        self.arena = PinnedArena(nbytes)
        self.stream = torch.cuda.Stream(self.device)  # default priority
        self._errors = _lib.DeviceErrors(self.device)
        self._batch = 0       # depth of open batches
        self._batch_wait = False

    @contextmanager
    def batch(self, ordered: bool = True):
        """Groups puts and gets: the copy stream waits for the current stream
        once on entry, and (``ordered``, or if the batch restored anything) the
        current stream waits for the copy stream once on exit, instead of a
        pair of waits per transfer."""
        if self._batch:
            self._batch += 1
            try:
                yield self
            finally:
                self._batch -= 1
            return
        cur = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(cur)
        self._batch, self._batch_wait = 1, ordered
        try:
            yield self
        finally:
            self._batch = 0
            if self._batch_wait:
                cur.wait_stream(self.stream)

    def _begin(self) -> torch.cuda.Stream:
        cur = torch.cuda.current_stream(self.device)
        if not self._batch:
            self.stream.wait_stream(cur)
        return cur

    def _end(self, cur: torch.cuda.Stream, wait: bool) -> None:
        if self._batch:
            self._batch_wait = self._batch_wait or wait
        elif wait:
            cur.wait_stream(self.stream)

    # ── dense tensors (DMA) ────────────────────────────────────────────────

    def put_tensor(self, t: torch.Tensor, off: int | None = None,
                   ordered: bool = True) -> HostTensor | None:
        """Starts the copy of a device tensor into the arena, at ``off`` (a
        range the caller holds) or in a new range; None if none fits.
        ``ordered``: later work on the current stream waits for the copy, so
        the source may be overwritten at once (the host never waits). Without
        it the copy overlaps that work, and the source must stay unchanged
        until ``sync``."""
        nbytes = t.numel() * t.element_size()
        if off is None:
            off = self.arena.alloc(nbytes)
            if off is None:
                return None
        src = t.detach().contiguous().view(-1).view(torch.uint8)
        cur = self._begin()
        with torch.cuda.stream(self.stream):
            self.arena.view(off, nbytes).copy_(src, non_blocking=True)
        src.record_stream(self.stream)
        self._end(cur, ordered)
        return HostTensor(off, nbytes, tuple(t.shape), t.dtype)

    def get_tensor(self, h: HostTensor) -> torch.Tensor:
        """A new device tensor with h's contents, ready on the current stream."""
        out = torch.empty(h.shape, dtype=h.dtype, device=self.device)
        cur = self._begin()
        with torch.cuda.stream(self.stream):
            out.view(-1).view(torch.uint8).copy_(self.arena.view(h.off, h.nbytes),
                                                  non_blocking=True)
        out.record_stream(self.stream)
        self._end(cur, True)
        return out

    # ── pool blocks (pack / unpack kernels across the host link) ──────────

    @staticmethod
    def blocks_bytes(pool: torch.Tensor, block_dims: int, n: int) -> int:
        planes, _, block_bytes, _ = pool_layout(pool, block_dims)
        return planes * n * block_bytes

    def put_blocks(self, pool: torch.Tensor, block_dims: int, ids: torch.Tensor,
                   off: int | None = None, ordered: bool = True) -> HostBlocks | None:
        """Starts packing blocks ``ids`` of every plane of ``pool`` into the
        arena, at ``off`` or in a new range; None if none fits. ``ordered`` as
        for ``put_tensor`` (the blocks may be reused at once)."""
        planes, stride, block_bytes, blocks = pool_layout(pool, block_dims)
        ids = self._ids(ids)
        n = ids.numel()
        nbytes = planes * n * block_bytes
        if off is None:
            off = self.arena.alloc(nbytes)
            if off is None:
                return None
        cur = self._begin()
        _lib.call("mkv_pack_blocks", pool.data_ptr(), stride, planes, block_bytes, blocks,
                  ids.data_ptr(), n, self.arena.buf.data_ptr() + off, self._errors.ptr(),
                  self.stream.cuda_stream)
        ids.record_stream(self.stream)
        self._end(cur, ordered)
        return HostBlocks(off, nbytes, planes, n, block_bytes)

    def get_blocks(self, h: HostBlocks, pool: torch.Tensor, block_dims: int,
                   ids: torch.Tensor) -> None:
        """Writes h's blocks into blocks ``ids`` (unique) of every plane of
        ``pool``; ordered before later work on the current stream."""
        planes, stride, block_bytes, blocks = pool_layout(pool, block_dims)
        ids = self._ids(ids)
        if (planes, ids.numel(), block_bytes) != (h.planes, h.n, h.block_bytes):
            raise ValueError(f"pool / ids ({planes} planes, {ids.numel()} blocks of "
                             f"{block_bytes} B) do not match the stored blocks "
                             f"({h.planes}, {h.n}, {h.block_bytes})")
        cur = self._begin()
        _lib.call("mkv_unpack_blocks", pool.data_ptr(), stride, planes, block_bytes, blocks,
                  ids.data_ptr(), h.n, self.arena.buf.data_ptr() + h.off, self._errors.ptr(),
                  self.stream.cuda_stream)
        ids.record_stream(self.stream)
        self._end(cur, True)

    def _ids(self, ids) -> torch.Tensor:
        """Block ids on the device, ready on the copy stream."""
        ids = torch.as_tensor(ids, dtype=torch.int32)
        if ids.device != self.device:  # uploaded on the copy stream itself
            with torch.cuda.stream(self.stream):
                return ids.contiguous().to(self.device, non_blocking=True)
        # device ids may come from the caller's stream after a batch began
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        return ids.contiguous()

    # ── lifetime ────────────────────────────────────────────────────────────

    def release(self, h: HostTensor | HostBlocks) -> None:
        """Returns h's range; later copies into it are ordered after every
        earlier use on the copy stream."""
        self.arena.free(h.off, h.nbytes)

    def sync(self) -> None:
        self.stream.synchronize()

    def check_errors(self) -> None:
        """Waits for the copy stream; raises MkvDeviceError on a bad block id."""
        self.stream.synchronize()
        self._errors.check("HostTier")
