"""Contiguous per-sequence KV cache — drop-in for muserve/memory/kv_cache.py.

``KVCache.append`` writes rows [current_len, current_len+n) of one attention
layer through the slot-mapped append kernel (the slots are a view of a cached
device arange, so an append is one launch and no allocation).
"""
from __future__ import annotations

import torch

from muserve_amd import _lib
from muserve_amd.config import ATTN_LAYER_INDICES

_ATTN_NUM_KV_HEADS = 2
_ATTN_HEAD_DIM = 256
_NUM_ATTN_LAYERS = 15
_ATTN_LAYER_INDICES = list(ATTN_LAYER_INDICES)


class KVCache:
    """Per-sequence KV cache for the 15 attention layers
    (muserve/memory/kv_cache.py:23-75): ``cache[15, 2, max_seq_len, 2, 256]``."""

    def __init__(self, max_seq_len: int, device: torch.device,
                 dtype: torch.dtype = torch.bfloat16):
        self.max_seq_len = max_seq_len
        self.device = device
        self.dtype = dtype
        self.current_len = 0
        self.cache = torch.zeros(_NUM_ATTN_LAYERS, 2, max_seq_len, _ATTN_NUM_KV_HEADS,
                                 _ATTN_HEAD_DIM, device=device, dtype=dtype)
        self._slots = None
        self._errors = None

    def _kernel_state(self):
        if self._slots is None:
            if self.cache.device.type != "cuda":
                raise RuntimeError(
                    f"KVCache on {self.cache.device}: the append kernel needs a ROCm GPU")
            self._slots = torch.arange(self.max_seq_len, dtype=torch.int64,
                                       device=self.cache.device)
            self._errors = _lib.DeviceErrors(self.cache.device)
        return self._slots

    def append(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor):
        """Appends k/v [num_new_tokens, num_kv_heads, head_dim] at current_len
        (advance() moves current_len once all layers are written)."""
        attn_idx = _ATTN_LAYER_INDICES.index(layer_idx)  # ValueError for a GDN layer
        num_new = k.shape[0]
        start = self.current_len
        end = start + num_new
        assert end <= self.max_seq_len, f"KV cache overflow: {end} > {self.max_seq_len}"
        slots = self._kernel_state()[start:end]
        row = _ATTN_NUM_KV_HEADS * _ATTN_HEAD_DIM
        k = k.to(device=self.cache.device, dtype=self.dtype).reshape(num_new, row).contiguous()
        v = v.to(device=self.cache.device, dtype=self.dtype).reshape(num_new, row).contiguous()
        if num_new == 0:
            return
        esz = self.cache.element_size()
        dev = self.cache.device
        _lib.call("mkv_append_bf16", self.cache[attn_idx, 0].data_ptr(),
                  self.cache[attn_idx, 1].data_ptr(), 0, self.max_seq_len, k.data_ptr(),
                  v.data_ptr(), 0, row * esz, slots.data_ptr(), num_new, 1, row * esz,
                  self._errors.ptr(), _lib.stream_of(dev))

    def get(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Views (k, v), each [current_len, num_kv_heads, head_dim]."""
        attn_idx = _ATTN_LAYER_INDICES.index(layer_idx)
        k = self.cache[attn_idx, 0, :self.current_len]
        v = self.cache[attn_idx, 1, :self.current_len]
        return k, v

    def advance(self, num_tokens: int):
        self.current_len += num_tokens

    def reset(self):
        self.current_len = 0

    @property
    def memory_bytes(self) -> int:
        return self.cache.numel() * self.cache.element_size()
