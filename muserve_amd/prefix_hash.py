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


def page_hashes_range(tokens: torch.Tensor, tok_offsets: torch.Tensor,
                      page_offsets: torch.Tensor, first: int, count: int, out: torch.Tensor,
                      errors: _lib.DeviceErrors) -> None:
    """Hashes requests first..first+count-1 with offsets already on the device
    (tok_offsets/page_offsets: int64 [R+1], global indices into tokens and
    out); no host work, no synchronisation."""
    if count <= 0:
        return
    if first < 0 or first + count + 1 > tok_offsets.numel() or \
            tok_offsets.numel() != page_offsets.numel():
        raise IndexError("request range outside the offset arrays")
    _lib.call("mkv_block_hash_sha256", tokens.data_ptr(), tok_offsets[first:].data_ptr(),
              page_offsets[first:].data_ptr(), count, tokens.element_size(), out.data_ptr(),
              errors.ptr(), _lib.stream_of(tokens.device))


def as_u64(h: torch.Tensor) -> np.ndarray:
    """Device int64 bit patterns -> host numpy uint64."""
    return h.cpu().numpy().view(np.uint64)
