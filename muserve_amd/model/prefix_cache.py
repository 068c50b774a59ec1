"""LRU prefix cache — drop-in for muserve/model/prefix_cache.py.

Keys, LRU order and eviction are the reference's (an OrderedDict keyed by
``sha256(ids as bytes).hexdigest()[:16]``, ``move_to_end`` on a hit or a
repeated store, ``popitem(last=False)`` when full). ``lookup`` gives the same
answer with less work: the ids cross to the host once, and all candidate
lengths are hashed in one incremental SHA-256 pass (a digest is taken at each
length in increasing order) instead of one device sync and one full hash
per cached entry.

SHA-256 over one prefix is a single dependent chain of compressions, which a
CPU core with SHA extensions runs far faster than one GPU lane; the GPU page
hasher (``block_manager.page_hashes``) pays off when many requests are hashed
in one launch.

Storage ``"cpu"`` of device tensors goes to a host tier
(muserve_amd/memory/host_tier.py) instead of ``tensor.cpu()`` /
``.to(device, non_blocking=True)`` (prefix_cache.py:36-44):
* an entry takes one range of a pinned arena;
* its tensors move by async DMA on a side stream, so ``store`` does not stall
  the caller;
* ``lookup`` restores into new device tensors ordered on the caller's stream.

When the arena cannot hold a new entry, entries leave in LRU order until it
fits; the reference evicts by count only. An entry may also carry the KV
pages of its prefix (``store(..., kv=(cache, page_ids))``), restored into
fresh pool pages by ``lookup_kv``; the reference keeps no KV. CPU tensors are
kept as the reference keeps them.
"""
from __future__ import annotations

import contextlib
import hashlib
from collections import OrderedDict
from typing import Optional

import torch

from muserve_amd.memory.host_tier import HostTensor, HostTier, PinnedArena

DEFAULT_HOST_BYTES = 4 << 30  # pinned arena of the "cpu" storage, allocated on first use


class PrefixCache:
    """LRU prefix cache of (hidden state, GDN states) with CPU or GPU storage."""

    def __init__(self, max_entries: int = 1024, storage: str = "cpu",
                 host_bytes: int = DEFAULT_HOST_BYTES, overlap_store: bool = False):
        """overlap_store: a store's copies overlap the caller's later GPU work
        instead of preceding it. The caller must then leave the stored tensors
        and pages unchanged until ``sync()``."""
        self.max_entries = max_entries
        self.storage = storage
        self.host_bytes = host_bytes
        self.overlap_store = overlap_store
        self._cache: OrderedDict[str, dict] = OrderedDict()
        self._tier: HostTier | None = None

    @staticmethod
    def _hash_tokens(token_ids: torch.Tensor) -> str:
        data = token_ids.cpu().numpy().tobytes()
        return hashlib.sha256(data).hexdigest()[:16]

    def _to_storage(self, tensor: torch.Tensor, off: int | None = None):
        if self.storage == "cpu":
            if tensor.device.type == "cuda":
                return self._tier.put_tensor(tensor, off, ordered=not self.overlap_store)
            return tensor.cpu()
        return tensor.clone()

    def _to_device(self, tensor, device: torch.device) -> torch.Tensor:
        if isinstance(tensor, HostTensor):
            out = self._tier.get_tensor(tensor)
            return out if out.device == device else out.to(device, non_blocking=True)
        if tensor.device != device:
            return tensor.to(device, non_blocking=True)
        return tensor

    @staticmethod
    def _prefix_keys(data: bytes, elem: int, lengths: list[int]) -> dict[int, str]:
        """Key of every prefix length (in tokens) in one incremental pass."""
        h = hashlib.sha256()
        done = 0
        keys = {}
        for n in sorted(set(lengths)):
            h.update(data[done * elem:n * elem])
            done = n
            keys[n] = h.copy().hexdigest()[:16]
        return keys

    def _find(self, input_ids: torch.Tensor) -> Optional[str]:
        """Key of the longest cached prefix of input_ids (the reference's scan,
        prefix_cache.py:54-66), or None."""
        n_ids = len(input_ids)
        cands = [e["prefix_len"] for e in self._cache.values() if e["prefix_len"] <= n_ids]
        if not cands:
            return None
        ids = input_ids.cpu().numpy()
        keys = self._prefix_keys(ids.tobytes(), ids.itemsize, cands)
        best_key = None
        best_len = 0
        for key, entry in self._cache.items():
            prefix_len = entry["prefix_len"]
            if prefix_len > n_ids or prefix_len <= best_len:
                continue
            if keys[prefix_len] == key:
                best_key = key
                best_len = prefix_len
        return best_key

    def lookup(self, input_ids: torch.Tensor,
               device: torch.device) -> Optional[tuple[int, torch.Tensor, list]]:
        """Longest cached prefix of input_ids: (prefix_len, hidden, gdn_states)
        moved to ``device`` (ordered on its current stream), or None."""
        key = self._find(input_ids)
        if key is None:
            return None
        self._cache.move_to_end(key)
        entry = self._cache[key]
        with self._batch(entry):
            hidden = self._to_device(entry["hidden"], device)
            gdn_states = [self._to_device(s, device) if s is not None else None
                          for s in entry["gdn_states"]]
        return entry["prefix_len"], hidden, gdn_states

    def _batch(self, entry: dict):
        """One copy-stream session for an entry's transfers (a no-op without
        the host tier)."""
        if self._tier is not None and "_range" in entry:
            return self._tier.batch(ordered=True)
        return contextlib.nullcontext()

    def lookup_kv(self, input_ids: torch.Tensor, device: torch.device, cache
                  ) -> Optional[tuple[int, torch.Tensor, list, Optional[list[int]]]]:
        """``lookup`` plus the entry's KV pages: pages taken from ``cache``
        (``alloc_pages``; raises on OOM, changing nothing) receive the stored
        K/V of every layer. Returns (prefix_len, hidden, gdn_states, page_ids),
        page_ids None if the entry holds no KV."""
        key = self._find(input_ids)
        if key is None:
            return None
        entry = self._cache[key]
        kv = entry.get("kv")
        pages = None
        if kv is not None:
            # (alloc_pages(0) would take every free page)
            pages = cache.alloc_pages(kv["n"]) if kv["n"] else []
        self._cache.move_to_end(key)
        # page ids go up on the caller's stream, before the copy stream is busy
        ids = torch.tensor(pages, dtype=torch.int32).to(device) if pages else None
        with self._batch(entry):
            if pages:
                self._tier.get_blocks(kv["pages"], cache.cache, 3, ids)
                if kv["scales"] is not None:
                    self._tier.get_blocks(kv["scales"], cache.scales, 2, ids)
            hidden = self._to_device(entry["hidden"], device)
            gdn_states = [self._to_device(s, device) if s is not None else None
                          for s in entry["gdn_states"]]
        return entry["prefix_len"], hidden, gdn_states, pages

    def store(self, input_ids: torch.Tensor, prefix_len: int, hidden: torch.Tensor,
              gdn_states: list, kv=None):
        """Caches the state after prefix_len tokens; evicts LRU entries when
        full. ``kv=(cache, page_ids)``: also keep the pages of ``cache`` that
        hold the prefix's K/V (all layers, and the fp8 scales)."""
        tensors = [hidden] + [s for s in gdn_states if s is not None]
        tiered = self.storage == "cpu" and any(t.device.type == "cuda" for t in tensors)
        if kv is not None and not tiered:
            raise ValueError("caching KV pages needs storage 'cpu' and device tensors")
        key = self._hash_tokens(input_ids[:prefix_len])
        if key in self._cache:
            self._cache.move_to_end(key)
            return
        while len(self._cache) >= self.max_entries:
            self._evict_lru()
        if not tiered:
            self._cache[key] = {
                "prefix_len": prefix_len,
                "hidden": self._to_storage(hidden),
                "gdn_states": [self._to_storage(s) if s is not None else None
                               for s in gdn_states],
            }
            return
        # one arena range for the whole entry (CPU tensors are kept as they are)
        if self._tier is None:
            self._tier = HostTier(self.host_bytes,
                                  next(t.device for t in tensors if t.device.type == "cuda"))
        sizes = [PinnedArena.rounded(t.numel() * t.element_size()) if t.device.type == "cuda"
                 else 0 for t in tensors]
        kv_sizes = []
        if kv is not None:
            cache, page_ids = kv
            n = len(page_ids)
            kv_sizes.append(PinnedArena.rounded(HostTier.blocks_bytes(cache.cache, 3, n)))
            if cache.scales is not None:
                kv_sizes.append(PinnedArena.rounded(HostTier.blocks_bytes(cache.scales, 2, n)))
        total = sum(sizes) + sum(kv_sizes)
        off = self._reserve(total)
        if off is None:
            return  # larger than the whole arena: not cached
        # page ids go up on the caller's stream, before the copy stream is busy
        kv_ids = (torch.as_tensor(kv[1], dtype=torch.int32).to(self._tier.device)
                  if kv is not None else None)
        with self._tier.batch(ordered=not self.overlap_store):
            self._store_parts(key, prefix_len, tensors, sizes, gdn_states, off, total, kv,
                              kv_sizes, kv_ids)

    def _store_parts(self, key, prefix_len, tensors, sizes, gdn_states, off, total, kv,
                     kv_sizes, ids):
        at = off
        stored = []
        for t, sz in zip(tensors, sizes):
            stored.append(self._to_storage(t, at) if sz else t.cpu())
            at += sz
        it = iter(stored)
        entry = {
            "prefix_len": prefix_len,
            "hidden": next(it),
            "gdn_states": [next(it) if s is not None else None for s in gdn_states],
            "_range": (off, total),
        }
        if kv is not None:
            cache, page_ids = kv
            n = len(page_ids)
            ordered = not self.overlap_store
            pages = self._tier.put_blocks(cache.cache, 3, ids, at, ordered)
            at += kv_sizes[0]
            scales = (self._tier.put_blocks(cache.scales, 2, ids, at, ordered)
                      if cache.scales is not None else None)
            entry["kv"] = {"n": n, "pages": pages, "scales": scales}
        self._cache[key] = entry

    def _reserve(self, nbytes: int) -> Optional[int]:
        if nbytes > self._tier.arena.nbytes:
            return None
        while True:
            off = self._tier.arena.alloc(nbytes)
            if off is not None or not self._cache:
                return off
            self._evict_lru()

    def _evict_lru(self) -> None:
        _, entry = self._cache.popitem(last=False)
        self._release(entry)

    def _release(self, entry: dict) -> None:
        rng = entry.get("_range")
        if rng is not None:
            self._tier.arena.free(*rng)

    def sync(self) -> None:
        """Waits until every started copy into or out of the host tier ended."""
        if self._tier is not None:
            self._tier.check_errors()

    def clear(self):
        for entry in self._cache.values():
            self._release(entry)
        self._cache.clear()

    def __len__(self):
        return len(self._cache)

    def memory_mb(self) -> float:
        total = 0
        for entry in self._cache.values():
            total += entry["hidden"].nelement() * entry["hidden"].element_size()
            for s in entry["gdn_states"]:
                if s is not None:
                    total += s.nelement() * s.element_size()
            kv = entry.get("kv")
            if kv is not None:
                total += kv["pages"].nbytes + (kv["scales"].nbytes if kv["scales"] else 0)
        return total / 1024 / 1024
