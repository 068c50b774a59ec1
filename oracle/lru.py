"""LRU prefix-cache model on the CPU (oracle; test infrastructure only).

PrefixCacheModel restates muserve/model/prefix_cache.py:46-105 over keys only
(no tensors): entries live in an OrderedDict in LRU order; a lookup scans them
in that order keeping the longest matching prefix (:57-66) and moves the hit
to the MRU end (:71); a store of a present key only moves it (:91-93);
otherwise LRU entries are popped until there is room (:95-96).
"""
from __future__ import annotations

from collections import OrderedDict

import numpy as np

from oracle.sha import hash_tokens


class PrefixCacheModel:
    def __init__(self, max_entries: int):
        self.max_entries = max_entries
        self.entries: OrderedDict[str, int] = OrderedDict()

    def lookup(self, ids: np.ndarray) -> int | None:
        best_key, best_len = None, 0
        for key, plen in self.entries.items():
            if plen > len(ids) or plen <= best_len:
                continue
            if hash_tokens(ids[:plen]) == key:
                best_key, best_len = key, plen
        if best_key is None:
            return None
        self.entries.move_to_end(best_key)
        return best_len

    def store(self, ids: np.ndarray, prefix_len: int) -> None:
        key = hash_tokens(ids[:prefix_len])
        if key in self.entries:
            self.entries.move_to_end(key)
            return
        while len(self.entries) >= self.max_entries:
            self.entries.popitem(last=False)
        self.entries[key] = prefix_len

    def keys(self) -> list[str]:
        return list(self.entries)
