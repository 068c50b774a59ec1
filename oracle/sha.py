"""Prefix hashes on the CPU with hashlib (oracle; test infrastructure only).

muserve/model/prefix_cache.py:31-34 keys a prefix by
sha256(ids.cpu().numpy().tobytes()).hexdigest()[:16]; the page hash of page i
is that key for the first 16*(i+1) tokens, as a big-endian u64.
"""
from __future__ import annotations

import hashlib

import numpy as np

PAGE = 16


def hash_tokens(ids: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(ids).tobytes()).hexdigest()[:16]


def key_u64(key: str) -> int:
    return int(key, 16)


def page_hashes(ids: np.ndarray) -> list[int]:
    """One incremental SHA-256 pass; a digest copy at every page boundary."""
    ids = np.ascontiguousarray(ids)
    h = hashlib.sha256()
    out = []
    for i in range(len(ids) // PAGE):
        h.update(ids[i * PAGE:(i + 1) * PAGE].tobytes())
        out.append(int(h.copy().hexdigest()[:16], 16))
    return out


def page_hashes_from_scratch(ids: np.ndarray) -> list[int]:
    """Each page's prefix hashed from scratch (quadratic; small cases only)."""
    return [key_u64(hash_tokens(ids[:PAGE * (i + 1)])) for i in range(len(ids) // PAGE)]
