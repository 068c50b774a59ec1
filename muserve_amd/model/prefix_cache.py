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
"""
from __future__ import annotations

import hashlib
from collections import OrderedDict
from typing import Optional

import torch


class PrefixCache:
    """LRU prefix cache of (hidden state, GDN states) with CPU or GPU storage."""

    def __init__(self, max_entries: int = 1024, storage: str = "cpu"):
        self.max_entries = max_entries
        self.storage = storage
        self._cache: OrderedDict[str, dict] = OrderedDict()

    @staticmethod
    def _hash_tokens(token_ids: torch.Tensor) -> str:
        data = token_ids.cpu().numpy().tobytes()
        return hashlib.sha256(data).hexdigest()[:16]

    def _to_storage(self, tensor: torch.Tensor) -> torch.Tensor:
        if self.storage == "cpu":
            return tensor.cpu()
        return tensor.clone()

    def _to_device(self, tensor: torch.Tensor, device: torch.device) -> torch.Tensor:
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

    def lookup(self, input_ids: torch.Tensor,
               device: torch.device) -> Optional[tuple[int, torch.Tensor, list]]:
        """Longest cached prefix of input_ids: (prefix_len, hidden, gdn_states)
        moved to ``device`` (non_blocking), or None."""
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
        if best_key is None:
            return None
        self._cache.move_to_end(best_key)
        entry = self._cache[best_key]
        hidden = self._to_device(entry["hidden"], device)
        gdn_states = [self._to_device(s, device) if s is not None else None
                      for s in entry["gdn_states"]]
        return best_len, hidden, gdn_states

    def store(self, input_ids: torch.Tensor, prefix_len: int, hidden: torch.Tensor,
              gdn_states: list):
        """Caches the state after prefix_len tokens; evicts LRU entries when full."""
        key = self._hash_tokens(input_ids[:prefix_len])
        if key in self._cache:
            self._cache.move_to_end(key)
            return
        while len(self._cache) >= self.max_entries:
            self._cache.popitem(last=False)
        self._cache[key] = {
            "prefix_len": prefix_len,
            "hidden": self._to_storage(hidden),
            "gdn_states": [self._to_storage(s) if s is not None else None for s in gdn_states],
        }

    def clear(self):
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
        return total / 1024 / 1024
