"""Paged KV-cache pool on gfx950 kernels — drop-in for muserve/kv_cache.py.

Pool layout (unchanged from muserve/kv_cache.py:4-10,45-49):
``cache[num_layers, 2, num_pages, page_size=16, kv_heads, head_dim]`` with
dim 1 = (K, V). One page of one (layer, K|V) plane is 16 contiguous token
rows (8 KiB for one bf16 head of 256), the unit every kernel streams.

``PagedKVCache`` and ``SequenceKVState`` keep the reference's signatures,
attribute names, allocation order and error types. New, additive APIs:

* ``PagedKVCache.append`` — slot-mapped append of any number of tokens for one
  or all layers in one launch (``write_kv`` is a thin wrapper over it);
* ``PagedKVCache.gather`` — block-table gather into padded ``[B, S, H, D]``
  or packed varlen rows, one launch for one or all layers;
* ``PagedKVCache.copy_pages`` — page copies for copy-on-write;
* fp8 e4m3fn pools (``dtype=torch.float8_e4m3fn``): ``append``/``write_kv``
  quantise bf16 input per (token, head) and ``gather`` dequantises to bf16;
* ``BlockTables`` — device-resident block tables and lengths for a batch of
  ``SequenceKVState`` with a one-launch decode step.
"""
from __future__ import annotations

import numpy as np
import torch

from muserve_amd import _lib
from muserve_amd.config import HEAD_DIM, KV_DTYPE, KV_PAGE_SIZE, NUM_KV_HEADS, NUM_LAYERS, TP_SIZE

_DTYPE_MAP = {
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "float8_e4m3fn": torch.float8_e4m3fn,
}
_FP8 = torch.float8_e4m3fn
_SIXTEEN_BIT = (torch.float16, torch.bfloat16)


def get_tp_rank() -> int:
    """Tensor-parallel rank (muserve/distributed.py:49-50); 0 without a group."""
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        return torch.distributed.get_rank()
    return 0


def _as_index(x, device: torch.device) -> torch.Tensor:
    """int / sequence / slice / tensor index -> int64 device tensor."""
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=torch.int64).reshape(-1)
    if isinstance(x, slice):
        return torch.arange(x.start or 0, x.stop, x.step or 1, dtype=torch.int64, device=device)
    if isinstance(x, (int, np.integer)):
        return torch.tensor([int(x)], dtype=torch.int64, device=device)
    return torch.as_tensor(np.asarray(x, dtype=np.int64), device=device).reshape(-1)


class PagedKVCache:
    """GPU paged KV cache with dynamic page allocation (muserve/kv_cache.py:25-118)."""

    def __init__(self, num_gpu_pages: int | None = None, *, num_layers: int = NUM_LAYERS,
                 kv_heads: int | None = None, head_dim: int = HEAD_DIM,
                 dtype: torch.dtype | None = None, device: torch.device | str | None = None,
                 verbose: bool = True):
        rank = get_tp_rank()
        device = torch.device(device) if device is not None else torch.device(f"cuda:{rank}")
        dtype = dtype if dtype is not None else _DTYPE_MAP[KV_DTYPE]
        if dtype not in (*_SIXTEEN_BIT, _FP8):
            raise ValueError(f"unsupported KV dtype {dtype}")
        # KV heads split across TP ranks, at least one per rank (muserve/kv_cache.py:34)
        kv_heads_per_rank = kv_heads if kv_heads is not None else max(1, NUM_KV_HEADS // TP_SIZE)

        if num_gpu_pages is None:
            num_gpu_pages = self._estimate_pages(device, kv_heads_per_rank, dtype, num_layers,
                                                 head_dim)

        self.num_pages = num_gpu_pages
        self.page_size = KV_PAGE_SIZE
        self.device = device
        self.num_layers = num_layers
        self.kv_heads = kv_heads_per_rank
        self.head_dim = head_dim
        self.dtype = dtype

        self.cache = torch.zeros(num_layers, 2, num_gpu_pages, KV_PAGE_SIZE, kv_heads_per_rank,
                                 head_dim, dtype=dtype, device=device)
        # fp8 pools carry one fp32 scale per (token, head): [L, 2, P, 16, H]
        self.scales = (torch.zeros(num_layers, 2, num_gpu_pages, KV_PAGE_SIZE, kv_heads_per_rank,
                                   dtype=torch.float32, device=device)
                       if dtype == _FP8 else None)

        # free-page stack, LIFO (muserve/kv_cache.py:51-53)
        self._free_pages = list(range(num_gpu_pages))
        self._num_free = num_gpu_pages
        self._errors = _lib.DeviceErrors(device) if device.type == "cuda" else None
        # opt-in: report a slot that appears twice in one append (MkvDeviceError)
        self.check_unique = _lib.CHECK_UNIQUE_DEFAULT
        self._unique: _lib.UniqueCheck | None = None

        if rank == 0 and verbose:
            nbytes = self.cache.numel() * self.cache.element_size()
            if self.scales is not None:
                nbytes += self.scales.numel() * 4
            print(f"[kv_cache] Allocated {num_gpu_pages} pages "
                  f"({nbytes / 1e9:.1f} GB, {kv_heads_per_rank} kv_heads/rank)")

    @staticmethod
    def _estimate_pages(device, kv_heads_per_rank: int, dtype: torch.dtype,
                        num_layers: int = NUM_LAYERS, head_dim: int = HEAD_DIM) -> int:
        """Pages that fit in 90 % of free HBM (muserve/kv_cache.py:60-73), with
        the element size taken from the dtype and fp8 scales counted."""
        free_bytes = torch.cuda.mem_get_info(device)[0]
        available = free_bytes - int(free_bytes * 0.10)
        elem = torch.empty((), dtype=dtype).element_size()
        per_token_head = head_dim * elem + (4 if dtype == _FP8 else 0)
        page_bytes = num_layers * 2 * KV_PAGE_SIZE * kv_heads_per_rank * per_token_head
        return int(max(1024, available // page_bytes))

    # ── allocation (muserve/kv_cache.py:77-98) ────────────────────────────────

    def alloc_pages(self, n: int) -> list[int]:
        """Pops n pages from the end of the free list, in list order; raises
        RuntimeError on OOM before any change. As in the reference, n == 0
        takes the whole list (``free[-0:]``) without changing the count."""
        if n > self._num_free:
            raise RuntimeError(
                f"KV cache OOM: requested {n} pages, only {self._num_free} free")
        pages = self._free_pages[-n:]
        del self._free_pages[-n:]
        self._num_free -= n
        return pages

    def free_pages(self, page_ids: list[int]) -> None:
        """Pushes pages back (no range or double-free check, as the reference)."""
        self._free_pages.extend(page_ids)
        self._num_free += len(page_ids)

    @property
    def num_free_pages(self) -> int:
        return self._num_free

    def num_free_tokens(self) -> int:
        return self._num_free * self.page_size

    def reserve_range(self, lo: int, hi: int) -> None:
        """Takes pages [lo, hi) out of the free list for good (the others keep
        their order): a block manager that owns those pages hands them out
        itself. All of them must be free."""
        if not 0 <= lo <= hi <= self.num_pages:
            raise ValueError(f"page range [{lo}, {hi}) outside the pool of {self.num_pages}")
        keep = [p for p in self._free_pages if not lo <= p < hi]
        if len(self._free_pages) - len(keep) != hi - lo:
            raise RuntimeError(f"pages [{lo}, {hi}) are not all free")
        self._free_pages = keep
        self._num_free = len(keep)

    def shuffle_free_list(self, generator: torch.Generator) -> None:
        """Replaces the free list by a seeded permutation of the free pages."""
        perm = torch.randperm(len(self._free_pages), generator=generator).tolist()
        self._free_pages = [self._free_pages[i] for i in perm]

    # ── geometry helpers ───────────────────────────────────────────────────────

    @property
    def num_slots(self) -> int:
        return self.num_pages * KV_PAGE_SIZE

    @property
    def row_elems(self) -> int:
        return self.kv_heads * self.head_dim

    def _plane_layer_stride(self) -> int:
        return 2 * self.num_slots * self.row_elems * self.cache.element_size()

    def _scale_layer_stride(self) -> int:
        return 2 * self.num_slots * self.kv_heads * 4

    def _gpu(self) -> torch.device:
        if self.device.type != "cuda":
            raise RuntimeError(
                f"PagedKVCache on {self.device}: the append/gather kernels need a ROCm GPU")
        return self.device

    def check_errors(self) -> None:
        """Synchronises and raises MkvDeviceError if a kernel flagged bad ids."""
        if self._errors is not None:
            self._errors.check("PagedKVCache")

    # ── KV write / read ────────────────────────────────────────────────────────

    def write_kv(self, layer_idx: int, page_idx, slot, k: torch.Tensor, v: torch.Tensor) -> None:
        """``cache[layer,0,page,slot] = k; cache[layer,1,page,slot] = v``
        (muserve/kv_cache.py:102-112). page_idx/slot may be ints, index tensors
        or (slot only) a slice; page[i] pairs with slot[i]. k/v hold
        [tokens, kv_heads, head_dim] (leading size-1 dims and broadcasting as
        in torch assignment). Runs the slot-mapped append kernel."""
        dev = self._gpu()
        pages = _as_index(page_idx, dev)
        slots = _as_index(slot, dev)
        pages, slots = torch.broadcast_tensors(pages, slots)
        slot_mapping = (pages * KV_PAGE_SIZE + slots).contiguous()
        n = slot_mapping.numel()
        self.append(slot_mapping, self._rows(k, n), self._rows(v, n), layer=layer_idx)

    def _rows(self, x: torch.Tensor, n: int) -> torch.Tensor:
        shape = (n, self.kv_heads, self.head_dim)
        if x.numel() != n * self.row_elems:
            x = x.expand(shape)
        return x.reshape(shape)

    def append(self, slot_mapping: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               layer: int | None = None) -> None:
        """Slot-mapped append. ``slot_mapping`` [T] int64 (slot = page*16 +
        offset; -1 skips a token); k/v [T, H, D] for ``layer``, or
        [L, T, H, D] for layers 0..L-1 when ``layer`` is None. Slots must be
        unique (with ``check_unique`` set, a repeat is reported as
        MkvDeviceError at the next ``check_errors``). For an fp8 pool k/v are
        bf16 and are quantised on the way in."""
        dev = self._gpu()
        if slot_mapping.dtype != torch.int64 or slot_mapping.device != dev:
            slot_mapping = slot_mapping.to(device=dev, dtype=torch.int64)
        slot_mapping = slot_mapping.contiguous()
        T = slot_mapping.numel()
        if layer is None:
            L = k.shape[0]
            first = 0
            if not (0 < L <= self.num_layers):
                raise ValueError(f"k holds {L} layers, pool has {self.num_layers}")
        else:
            L, first = 1, int(layer)
            if not (-self.num_layers <= first < self.num_layers):
                raise IndexError(f"layer {layer} out of range for {self.num_layers} layers")
            first %= self.num_layers
            k, v = k.unsqueeze(0), v.unsqueeze(0)
        want = (L, T, self.kv_heads, self.head_dim)
        if tuple(k.shape) != want or tuple(v.shape) != want:
            raise ValueError(f"k/v must be {want}, got {tuple(k.shape)} / {tuple(v.shape)}")
        in_dtype = torch.bfloat16 if self.dtype == _FP8 else self.dtype
        k = k.to(device=dev, dtype=in_dtype).contiguous()
        v = v.to(device=dev, dtype=in_dtype).contiguous()
        _lib.require_gpu(k, v, slot_mapping, self.cache)
        if T == 0:
            return
        if self.check_unique:
            if self._unique is None:
                self._unique = _lib.UniqueCheck(dev, self.num_slots)
            self._unique.run(slot_mapping, self._errors)
        esz = self.cache.element_size()
        kp = self.cache[first, 0]
        vp = self.cache[first, 1]
        src_layer = T * self.row_elems * 2
        src_tok = self.row_elems * 2
        stream = _lib.stream_of(dev)
        if self.dtype == _FP8:
            _lib.call("mkv_append_fp8", kp.data_ptr(), vp.data_ptr(),
                      self.scales[first, 0].data_ptr(), self.scales[first, 1].data_ptr(),
                      self._plane_layer_stride(), self._scale_layer_stride(), self.num_slots,
                      k.data_ptr(), v.data_ptr(), src_layer, src_tok, slot_mapping.data_ptr(), T,
                      L, self.kv_heads, self.head_dim, self._errors.ptr(), stream)
        else:
            _lib.call("mkv_append_bf16", kp.data_ptr(), vp.data_ptr(), self._plane_layer_stride(),
                      self.num_slots, k.data_ptr(), v.data_ptr(), src_layer, src_tok,
                      slot_mapping.data_ptr(), T, L, self.row_elems * esz, self._errors.ptr(),
                      stream)

    def get_kv_by_layer(self, layer_idx: int):
        """(k_cache, v_cache) views [num_pages, 16, kv_heads, head_dim]
        (muserve/kv_cache.py:114-118), as flash_attn_with_kvcache reads them."""
        return self.cache[layer_idx, 0], self.cache[layer_idx, 1]

    def gather(self, layer: int | None, block_tables: torch.Tensor, seq_lens: torch.Tensor,
               out_len: int | None = None, starts: torch.Tensor | None = None,
               out: tuple[torch.Tensor, torch.Tensor] | None = None,
               cu_out: torch.Tensor | None = None, num_layers: int | None = None):
        """Block-table gather into contiguous per-sequence K/V.

        block_tables [B, W] int32 page ids, seq_lens [B] int32, starts [B] int32
        (optional window start per sequence). Padded mode (``cu_out`` None)
        returns (k, v) of shape [B, out_len, H, D] with rows past a sequence's
        end zero — the [B,S,H,D] decode layout of
        muserve/model/qwen35_model.py:223-249. Packed mode writes sequence b's
        rows at ``cu_out[b]`` of [total, H, D] buffers (``cu_out`` holds B+1
        offsets; a sequence whose window does not fit between ``cu_out[b]`` and
        ``cu_out[b+1]``, or past the buffer's end, is cut there and flagged
        as MkvDeviceError at the next ``check_errors``). With ``layer`` None the
        first ``num_layers`` layers are gathered into [L, ...] outputs in one
        launch. fp8 pools are dequantised to bf16. ``out`` reuses buffers.
        """
        dev = self._gpu()
        B = block_tables.shape[0]
        if out_len is None:
            if cu_out is not None:
                raise ValueError("packed gather needs out_len (the longest window)")
            out_len = block_tables.shape[1] * KV_PAGE_SIZE
        if layer is None:
            L, first = (num_layers or self.num_layers), 0
        else:
            L, first = 1, int(layer) % self.num_layers
        if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
            raise TypeError("block_tables and seq_lens must be int32")
        if block_tables.stride(1) != 1:
            raise ValueError("block_tables rows must be contiguous")
        out_dtype = torch.bfloat16 if self.dtype == _FP8 else self.dtype
        rows = (B * out_len) if cu_out is None else None
        if cu_out is not None and cu_out.numel() != B + 1:
            raise ValueError("cu_out must hold B+1 offsets")
        if out is None:
            if cu_out is None:
                shape = (B, out_len, self.kv_heads, self.head_dim)
            else:
                shape = (max(0, int(cu_out[-1].item())), self.kv_heads, self.head_dim)
            if layer is None:
                shape = (L, *shape)
            k_out = torch.empty(shape, dtype=out_dtype, device=dev)
            v_out = torch.empty(shape, dtype=out_dtype, device=dev)
        else:
            k_out, v_out = out
            if k_out.dtype != out_dtype or v_out.dtype != out_dtype:
                raise TypeError(f"out buffers must be {out_dtype}")
            if not (k_out.is_contiguous() and v_out.is_contiguous()):
                raise ValueError("out buffers must be contiguous")
            if rows is not None and (k_out.numel() != L * rows * self.row_elems
                                     or v_out.numel() != k_out.numel()):
                raise ValueError(f"out buffers must hold exactly {L}x{rows} rows")
            if rows is None and (k_out.numel() % (L * self.row_elems) != 0
                                 or v_out.numel() != k_out.numel()):
                raise ValueError(f"packed out buffers must hold whole rows for {L} layers")
        _lib.require_gpu(block_tables, seq_lens, k_out, v_out, self.cache)
        if starts is not None:
            starts = starts.to(device=dev, dtype=torch.int32).contiguous()
        offs = None if cu_out is None else cu_out.to(device=dev, dtype=torch.int64).contiguous()
        seq_lens = seq_lens.contiguous()
        out_elem = 2
        out_layer_stride = (k_out.numel() // L) * out_elem
        stream = _lib.stream_of(dev)
        kp, vp = self.cache[first, 0], self.cache[first, 1]
        if self.dtype == _FP8:
            _lib.call("mkv_gather_dequant_fp8", kp.data_ptr(), vp.data_ptr(),
                      self.scales[first, 0].data_ptr(), self.scales[first, 1].data_ptr(),
                      self._plane_layer_stride(), self._scale_layer_stride(), self.num_pages,
                      block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
                      seq_lens.data_ptr(), _lib.ptr(starts), B, out_len, _lib.ptr(offs),
                      k_out.data_ptr(), v_out.data_ptr(), out_layer_stride, L, self.kv_heads,
                      self.head_dim, self._errors.ptr(), stream)
        else:
            _lib.call("mkv_gather_bf16", kp.data_ptr(), vp.data_ptr(), self._plane_layer_stride(),
                      self.num_pages, block_tables.data_ptr(), block_tables.stride(0),
                      block_tables.shape[1], seq_lens.data_ptr(), _lib.ptr(starts), B, out_len,
                      _lib.ptr(offs), k_out.data_ptr(), v_out.data_ptr(), out_layer_stride, L,
                      self.row_elems * self.cache.element_size(), self._errors.ptr(), stream)
        return k_out, v_out

    def copy_pages(self, src_pages, dst_pages) -> None:
        """For every pair, page dst := page src in all layers and both K and V
        (and the fp8 scales): the copy a copy-on-write fork needs. The dst set
        must not overlap the src set; a pair with a negative id is skipped."""
        dev = self._gpu()

        def ids(x):
            if isinstance(x, torch.Tensor) and x.dtype == torch.int32 and x.device == dev:
                return x.contiguous()
            return _as_index(x, dev).to(torch.int32).contiguous()

        src, dst = ids(src_pages), ids(dst_pages)
        if src.numel() != dst.numel():
            raise ValueError("src_pages and dst_pages differ in length")
        n = src.numel()
        if n == 0:
            return
        stream = _lib.stream_of(dev)
        page_bytes = KV_PAGE_SIZE * self.row_elems * self.cache.element_size()
        _lib.call("mkv_copy_blocks", self.cache.data_ptr(), self.num_pages * page_bytes,
                  2 * self.num_layers, self.num_pages, page_bytes, src.data_ptr(), dst.data_ptr(),
                  n, self._errors.ptr(), stream)
        if self.scales is not None:
            sbytes = KV_PAGE_SIZE * self.kv_heads * 4
            if sbytes % 16 == 0:
                _lib.call("mkv_copy_blocks", self.scales.data_ptr(), self.num_pages * sbytes,
                          2 * self.num_layers, self.num_pages, sbytes, src.data_ptr(),
                          dst.data_ptr(), n, self._errors.ptr(), stream)


class SequenceKVState:
    """One sequence's page table and length (muserve/kv_cache.py:121-158)."""

    def __init__(self, max_pages: int = 4096):
        self.page_table: list[int] = []
        self.seq_len: int = 0
        self.max_pages = max_pages

    @property
    def num_pages_used(self) -> int:
        return len(self.page_table)

    @property
    def last_page_slot(self) -> int:
        """Slot of the last token inside its page (0 when empty)."""
        if self.seq_len == 0:
            return 0
        return (self.seq_len - 1) % KV_PAGE_SIZE

    def needs_new_page(self) -> bool:
        """True when the next token starts a page."""
        if not self.page_table:
            return True
        return self.seq_len % KV_PAGE_SIZE == 0

    def current_page(self) -> int:
        return self.page_table[-1]

    def to_page_table_tensor(self, max_pages: int, device) -> torch.Tensor:
        """[1, max_pages] int32, unused entries 0 (muserve/kv_cache.py:149-158).
        Built on the host and copied once instead of one device write per page;
        a table longer than max_pages raises IndexError like the reference's
        out-of-range element write."""
        n = len(self.page_table)
        if n > max_pages:
            raise IndexError(
                f"index {max_pages} is out of bounds for dimension 1 with size {max_pages}")
        host = np.zeros((1, max_pages), dtype=np.int32)
        host[0, :n] = self.page_table
        return torch.from_numpy(host).to(device)


def slot_mapping_for(seq: SequenceKVState, start: int, n: int) -> np.ndarray:
    """Slots of token positions [start, start+n) of a sequence whose page table
    already covers them (slot = page*16 + position%16)."""
    pos = np.arange(start, start + n, dtype=np.int64)
    table = np.asarray(seq.page_table, dtype=np.int64)
    return table[pos // KV_PAGE_SIZE] * KV_PAGE_SIZE + pos % KV_PAGE_SIZE


def reserve_tokens(cache: PagedKVCache, seq: SequenceKVState, n: int) -> int:
    """Adds n tokens to a sequence's bookkeeping and returns their first
    position. Pages come from ``cache.alloc_pages`` exactly as the reference's
    per-token loop takes them (muserve/scripts/test_kv_cache.py:88-92: one
    ``alloc_pages(1)`` whenever a token starts a page), in one call."""
    start = seq.seq_len
    need = -(-(start + n) // KV_PAGE_SIZE) - len(seq.page_table)
    if n > 0 and need > 0:
        pages = cache.alloc_pages(need)
        seq.page_table.extend(reversed(pages))  # successive alloc_pages(1) pop from the end
    seq.seq_len += n
    return start


def prefill_slot_mapping(cache: PagedKVCache, seqs: list[SequenceKVState],
                         lengths: list[int]) -> torch.Tensor:
    """Reserves ``lengths[i]`` tokens on each sequence (``reserve_tokens``) and
    returns the concatenated int64 slot mapping on the cache's device."""
    parts = []
    for seq, n in zip(seqs, lengths):
        start = reserve_tokens(cache, seq, int(n))
        parts.append(slot_mapping_for(seq, start, int(n)))
    flat = np.concatenate(parts) if parts else np.zeros(0, dtype=np.int64)
    return torch.from_numpy(flat).to(cache.device)


class BlockTables:
    """Device block tables [B, max_pages] int32 and lengths [B] int32 for a
    batch of sequences, kept in step with their ``SequenceKVState`` objects.

    ``decode_step`` advances every sequence by one token: the host pops one
    page per sequence that starts a page — in batch order, the same pages
    repeated ``alloc_pages(1)`` calls return — and a single kernel writes the
    new table entries, produces the slot mapping and bumps the lengths.
    """

    _RING = 4  # pinned staging buffers in flight

    def __init__(self, cache: PagedKVCache, seqs: list[SequenceKVState], max_pages: int):
        self.cache = cache
        self.seqs = seqs
        dev = cache._gpu()
        B = len(seqs)
        host = np.zeros((B, max_pages), dtype=np.int32)
        lens = np.zeros(B, dtype=np.int32)
        for b, s in enumerate(seqs):
            if len(s.page_table) > max_pages:
                raise IndexError(f"sequence {b} holds {len(s.page_table)} pages > {max_pages}")
            host[b, :len(s.page_table)] = s.page_table
            lens[b] = s.seq_len
        self.max_pages = max_pages
        self.tables = torch.from_numpy(host).to(dev)
        self.seq_lens = torch.from_numpy(lens).to(dev)
        self._lens = lens.astype(np.int64)
        self.slots = torch.empty(B, dtype=torch.int64, device=dev)
        self._new_dev = torch.empty(B, dtype=torch.int32, device=dev)
        self._pinned = [torch.empty(B, dtype=torch.int32, pin_memory=True)
                        for _ in range(self._RING)]
        self._events = [None] * self._RING
        self._ring = 0

    @property
    def batch(self) -> int:
        return len(self.seqs)

    def decode_step(self) -> torch.Tensor:
        """One new token per sequence; returns the slot mapping [B] int64."""
        cache = self.cache
        dev = cache.device
        need = np.flatnonzero(self._lens % KV_PAGE_SIZE == 0)
        if need.size and int(self._lens[need].max()) // KV_PAGE_SIZE >= self.max_pages:
            raise IndexError("a sequence outgrew its block table")
        pages = cache.alloc_pages(int(need.size)) if need.size else []
        i = self._ring
        self._ring = (i + 1) % self._RING
        if self._events[i] is not None:
            self._events[i].synchronize()
        staging = self._pinned[i]
        buf = staging.numpy()
        buf.fill(-1)
        if need.size:
            # repeated alloc_pages(1): the first needy sequence takes the last page
            buf[need] = np.asarray(pages[::-1], dtype=np.int32)
            for b, p in zip(need.tolist(), pages[::-1]):
                self.seqs[b].page_table.append(p)
        for s in self.seqs:
            s.seq_len += 1
        self._lens += 1
        stream = _lib.stream_of(dev)
        self._new_dev.copy_(staging, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dev))
        self._events[i] = ev
        _lib.call("mkv_decode_slots", self.seq_lens.data_ptr(), self.tables.data_ptr(),
                  self.tables.stride(0), self.max_pages, self._new_dev.data_ptr(), self.batch,
                  cache.num_pages, self.slots.data_ptr(), cache._errors.ptr(), stream)
        return self.slots

    def padded_len(self) -> int:
        """Longest sequence rounded up to whole pages (the padded gather width)."""
        if not len(self._lens):
            return 0
        return int(-(-int(self._lens.max()) // KV_PAGE_SIZE) * KV_PAGE_SIZE)
