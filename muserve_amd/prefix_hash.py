"""Batched per-page prefix hashes on the GPU.

page i of a request is keyed by the first 8 bytes (big-endian) of SHA-256 over
its first 16*(i+1) token ids as little-endian integers — the prefix key of
muserve/model/prefix_cache.py:31-34 evaluated at every page boundary. One
kernel lane walks one request, so a launch should carry a batch of requests.
"""
from __future__ import annotations

import numpy as np
import torch

from muserve_amd import _lib
from muserve_amd.config import KV_PAGE_SIZE


def page_offsets(cu_tokens: np.ndarray) -> np.ndarray:
    """[R+1] token offsets -> [R+1] offsets of each request's full pages."""
    n = np.diff(np.asarray(cu_tokens, dtype=np.int64)) // KV_PAGE_SIZE
    return np.concatenate([[0], np.cumsum(n)]).astype(np.int64)


def page_hashes(tokens: torch.Tensor, cu_tokens, errors: _lib.DeviceErrors | None = None,
                out: torch.Tensor | None = None):
    """tokens: flat int64 (or int32) ids on the GPU; cu_tokens: [R+1] host
    offsets. Returns (hashes, cu_pages): hashes is an int64 device tensor
    holding each page hash's u64 bit pattern, cu_pages the host page offsets."""
    dev = _lib.require_gpu(tokens)
    if tokens.dtype not in (torch.int64, torch.int32):
        raise TypeError("token ids must be int64 or int32")
    cu_t = np.asarray(cu_tokens.cpu() if isinstance(cu_tokens, torch.Tensor) else cu_tokens,
                      dtype=np.int64)
    if cu_t[0] != 0 or (np.diff(cu_t) < 0).any() or cu_t[-1] > tokens.numel():
        raise ValueError("cu_tokens must be non-decreasing offsets into tokens starting at 0")
    cu_p = page_offsets(cu_t)
    total = int(cu_p[-1])
    if out is None:
        out = torch.empty(total, dtype=torch.int64, device=dev)
    elif out.numel() < total or out.dtype != torch.int64:
        raise ValueError("out must be an int64 tensor with room for every page hash")
    R = len(cu_t) - 1
    if R == 0:
        return out[:0], cu_p
    tokens = tokens.contiguous()
    dev_offs = torch.from_numpy(np.concatenate([cu_t, cu_p])).to(dev, non_blocking=False)
    err = errors or _lib.DeviceErrors(dev)
    _lib.call("mkv_block_hash_sha256", tokens.data_ptr(), dev_offs.data_ptr(),
              dev_offs[R + 1:].data_ptr(), R, tokens.element_size(), out.data_ptr(), err.ptr(),
              _lib.stream_of(dev))
    if errors is None:
        err.check("page_hashes")
    return out[:total], cu_p


def as_u64(h: torch.Tensor) -> np.ndarray:
    """Device int64 bit patterns -> host numpy uint64."""
    return h.cpu().numpy().view(np.uint64)
