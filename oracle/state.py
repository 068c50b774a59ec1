"""GDN state-pool slot moves on the CPU (oracle; test infrastructure only).

The reference keeps per-request state tensors (muserve/model/qwen35_model.py:
28-49,94-126); a slot pool's batch gather is pool[layer][slots] and its
scatter pool[layer][slots] = x.
"""
from __future__ import annotations

import torch


def gather(pool: torch.Tensor, layer: int, slots: torch.Tensor) -> torch.Tensor:
    return pool[layer].index_select(0, slots.to(torch.int64))


def scatter(pool: torch.Tensor, layer: int, slots: torch.Tensor, x: torch.Tensor) -> None:
    pool[layer].index_copy_(0, slots.to(torch.int64), x)


def pack_blocks(pool: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """Host-tier pack of a layered pool [planes, blocks, ...]: every plane's
    blocks ids, plane-major -> [planes, n, ...]. An id outside the pool gives
    zeros. Replaces the per-tensor `.cpu()` of PrefixCache._to_storage
    (muserve/model/prefix_cache.py:36-39) for state kept in a pool."""
    ids = ids.to(torch.int64)
    ok = (ids >= 0) & (ids < pool.shape[1])
    out = pool.index_select(1, torch.where(ok, ids, torch.zeros_like(ids)))
    out[:, ~ok] = 0
    return out


def unpack_blocks(pool: torch.Tensor, ids: torch.Tensor, packed: torch.Tensor) -> None:
    """The inverse (PrefixCache._to_device, prefix_cache.py:41-44): pool
    [:, ids[i]] = packed[:, i]; ids outside the pool are skipped."""
    ids = ids.to(torch.int64)
    ok = (ids >= 0) & (ids < pool.shape[1])
    pool.index_copy_(1, ids[ok], packed[:, ok])
