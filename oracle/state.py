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
