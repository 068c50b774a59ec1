"""Paged pool, page tables and gathers on the CPU (oracle; test infrastructure only).

Everything is a restatement of muserve/kv_cache.py and of the decode-time
contiguous K/V layout of muserve/model/qwen35_model.py:223-249 and
muserve/model/qwen35_layer_v2.py:485-492.
"""
from __future__ import annotations

import numpy as np
import torch

PAGE = 16  # muserve/config.py:36


class PoolModel:
    """Free-page list of PagedKVCache (muserve/kv_cache.py:52-53,77-98)."""

    def __init__(self, num_pages: int, free_list: list[int] | None = None):
        self.free = list(range(num_pages)) if free_list is None else list(free_list)
        self.num_free = len(self.free)

    def alloc(self, n: int) -> list[int]:
        # muserve/kv_cache.py:77-86
        if n > self.num_free:
            raise RuntimeError(f"KV cache OOM: requested {n} pages, only {self.num_free} free")
        pages = self.free[-n:]
        del self.free[-n:]
        self.num_free -= n
        return pages

    def release(self, pages: list[int]) -> None:
        # muserve/kv_cache.py:88-91
        self.free.extend(pages)
        self.num_free += len(pages)


class SeqModel:
    """SequenceKVState (muserve/kv_cache.py:121-158)."""

    def __init__(self):
        self.page_table: list[int] = []
        self.seq_len = 0

    def last_page_slot(self) -> int:
        return 0 if self.seq_len == 0 else (self.seq_len - 1) % PAGE   # :133-138

    def needs_new_page(self) -> bool:
        return (not self.page_table) or self.seq_len % PAGE == 0       # :140-144

    def add_tokens(self, pool: PoolModel, n: int) -> list[int]:
        """The per-token loop of muserve/scripts/test_kv_cache.py:88-92; returns
        the slot (page*16 + offset) of every added token."""
        slots = []
        for _ in range(n):
            if self.needs_new_page():
                self.page_table.append(pool.alloc(1)[0])
            slots.append(self.page_table[self.seq_len // PAGE] * PAGE + self.seq_len % PAGE)
            self.seq_len += 1
        return slots


def page_table_tensor(page_table: list[int], max_pages: int) -> torch.Tensor:
    """muserve/kv_cache.py:149-158: zeros, then element writes (IndexError past the end)."""
    t = torch.zeros(1, max_pages, dtype=torch.int32)
    for i, p in enumerate(page_table):
        t[0, i] = p
    return t


def write_kv(cache: torch.Tensor, layer: int, page, slot, k: torch.Tensor, v: torch.Tensor):
    """muserve/kv_cache.py:111-112 on a CPU pool [L, 2, P, 16, H, D]."""
    cache[layer, 0, page, slot] = k
    cache[layer, 1, page, slot] = v


def append(cache: torch.Tensor, slot_mapping: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
           layer: int | None = None):
    """Slot-mapped append: write_kv with page = slot // 16, offset = slot % 16
    for every token whose slot is not -1. k/v: [T,H,D] (one layer) or [L,T,H,D]."""
    slot_mapping = slot_mapping.to(torch.int64)
    keep = slot_mapping >= 0
    pages = slot_mapping[keep] // PAGE
    offs = slot_mapping[keep] % PAGE
    layers = [layer] if layer is not None else list(range(k.shape[0]))
    for i, l in enumerate(layers):
        kk = k if layer is not None else k[i]
        vv = v if layer is not None else v[i]
        write_kv(cache, l, pages, offs, kk[keep], vv[keep])


def gather_padded(plane: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
                  out_len: int, starts: torch.Tensor | None = None) -> torch.Tensor:
    """Contiguous [B, out_len, H, D] rows of one (layer, K|V) plane
    [P, 16, H, D]: row i of sequence b is position starts[b]+i if it is below
    seq_lens[b], else zeros — the [B,S,H,D] layout decode attention reads
    (muserve/model/qwen35_model.py:246-247)."""
    P, page, H, D = plane.shape
    rows = plane.reshape(P * page, H, D)
    B = block_tables.shape[0]
    out = torch.zeros(B, out_len, H, D, dtype=plane.dtype)
    bt = block_tables.to(torch.int64)
    for b in range(B):
        s = int(starts[b]) if starts is not None else 0
        n = max(0, min(int(seq_lens[b]) - s, out_len))
        if n == 0:
            continue
        pos = torch.arange(s, s + n)
        slots = bt[b, pos // PAGE] * PAGE + pos % PAGE
        out[b, :n] = rows.index_select(0, slots)
    return out


def gather_packed(plane: torch.Tensor, block_tables: torch.Tensor,
                  seq_lens: torch.Tensor) -> list[torch.Tensor]:
    """Each sequence back to contiguous [len, H, D]."""
    P, page, H, D = plane.shape
    rows = plane.reshape(P * page, H, D)
    out = []
    bt = block_tables.to(torch.int64)
    for b in range(bt.shape[0]):
        pos = torch.arange(int(seq_lens[b]))
        out.append(rows.index_select(0, bt[b, pos // PAGE] * PAGE + pos % PAGE))
    return out


def gather_bruteforce(plane: np.ndarray, block_tables: np.ndarray, seq_lens: np.ndarray,
                      out_len: int, starts: np.ndarray | None = None) -> np.ndarray:
    """Independent per-position restatement (pure Python loops; small cases only)."""
    P, page, H, D = plane.shape
    B = block_tables.shape[0]
    out = np.zeros((B, out_len, H, D), dtype=plane.dtype)
    for b in range(B):
        s = int(starts[b]) if starts is not None else 0
        for i in range(out_len):
            p = s + i
            if p < int(seq_lens[b]):
                out[b, i] = plane[block_tables[b][p // page], p % page]
    return out


def decode_step(pool: PoolModel, seqs: list[SeqModel]) -> list[int]:
    """One decode token for every sequence in batch order: a sequence that
    starts a page takes alloc(1) (the test_kv_cache.py:88-92 pattern); returns
    the slot mapping."""
    return [s.add_tokens(pool, 1)[0] for s in seqs]
