"""Slot pool for GDN linear-attention states (recurrent + conv), per rank.

The reference threads GDN states through the model as per-request,
per-layer tensors (muserve/model/qwen35_model.py:28-49,94-126; the
``.contiguous()`` of muserve/inference_loop.py:108). For continuous batching
this module keeps them resident in two pools indexed by a request slot:

* recurrent ``state[L_gdn, num_slots, v_heads, v_dim, k_dim]`` fp32 — the
  "VK" layout the decode kernel reads (muserve/model/qwen35_layer_v2.py:293),
  8 heads x 128 x 128 per rank = 512 KiB per (layer, slot);
* conv ``conv[L_gdn, num_slots, channels, width]`` bf16 (2048 x 4 = 16 KiB).

``gather(layer, slots)`` copies a batch's entries into contiguous buffers and
``scatter`` writes updated entries back, both layer's pools in one launch.
Slot ids within a ``scatter`` (and ``reset``, ``conv_decode``,
``decode_gather``) must be unique; with ``check_unique`` set a repeat is
reported as MkvDeviceError at the next ``check_errors``.
"""
from __future__ import annotations

import torch

from muserve_amd import _lib
from muserve_amd.config import GDN_CONV_KERNEL, GDN_KEY_DIM, GDN_VALUE_DIM

GDN_V_HEADS_PER_RANK = 8   # 64 value heads / TP 8 (muserve/model/qwen35_layer_v2.py:46-47)
CONV_CHANNELS_PER_RANK = 2048


def gdn_ordinal(layer_idx: int) -> int:
    """Index of a GDN layer among the 45 GDN layers of the 60-layer stack
    (attention layers are those with layer % 4 == 3)."""
    if layer_idx % 4 == 3:
        raise ValueError(f"layer {layer_idx} is an attention layer")
    return layer_idx - (layer_idx + 1) // 4


class StatePool:
    def __init__(self, num_layers: int = 45, num_slots: int = 1024,
                 state_shape: tuple[int, ...] = (GDN_V_HEADS_PER_RANK, GDN_VALUE_DIM, GDN_KEY_DIM),
                 state_dtype: torch.dtype = torch.float32,
                 conv_shape: tuple[int, ...] | None = (CONV_CHANNELS_PER_RANK, GDN_CONV_KERNEL),
                 conv_dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda"):
        self.device = torch.device(device)
        self.num_layers = num_layers
        self.num_slots = num_slots
        self.state = torch.zeros(num_layers, num_slots, *state_shape, dtype=state_dtype,
                                 device=self.device)
        self.conv = (torch.zeros(num_layers, num_slots, *conv_shape, dtype=conv_dtype,
                                 device=self.device) if conv_shape is not None else None)
        self._free = list(range(num_slots))
        self._errors = _lib.DeviceErrors(self.device) if self.device.type == "cuda" else None
        # opt-in: report a slot that appears twice where slots must be unique
        # (scatter, reset, the in-place conv) as MkvDeviceError
        self.check_unique = _lib.CHECK_UNIQUE_DEFAULT
        self._unique: _lib.UniqueCheck | None = None

    # slot bookkeeping: a LIFO stack, like the KV page free list
    def alloc_slot(self) -> int:
        if not self._free:
            raise RuntimeError(f"state pool full: all {self.num_slots} slots in use")
        return self._free.pop()

    def free_slot(self, slot: int) -> None:
        self._free.append(slot)

    @property
    def num_free_slots(self) -> int:
        return len(self._free)

    def _entry_bytes(self, t: torch.Tensor) -> int:
        return t[0, 0].numel() * t.element_size()

    def _check(self, slots: torch.Tensor, unique: bool = False) -> torch.Tensor:
        if self.device.type != "cuda":
            raise RuntimeError(f"StatePool on {self.device}: the slot kernels need a ROCm GPU")
        if slots.dtype != torch.int32 or slots.device != self.device:
            slots = slots.to(device=self.device, dtype=torch.int32)
        slots = slots.contiguous()
        if unique and self.check_unique:
            if self._unique is None:
                self._unique = _lib.UniqueCheck(self.device, self.num_slots)
            self._unique.run(slots, self._errors)
        return slots

    def reset(self, slots) -> None:
        """Zeroes the recurrent and conv states of ``slots`` in every layer, the
        zero initial states a new request starts from (``_init_gdn_states`` /
        ``_init_conv_states``, muserve/model/qwen35_model.py:28-49), for slots
        reused across requests. Slots must be unique; one launch per pool."""
        if not isinstance(slots, torch.Tensor):
            slots = torch.as_tensor(list(slots), dtype=torch.int32)
        slots = self._check(slots, unique=True)
        n = slots.numel()
        if n == 0:
            return
        for pool in (self.state, self.conv):
            if pool is None:
                continue
            _lib.call("mkv_zero_blocks", pool.data_ptr(), pool.stride(0) * pool.element_size(),
                      self.num_layers, self._entry_bytes(pool), self.num_slots, slots.data_ptr(),
                      n, self._errors.ptr(), _lib.stream_of(self.device))

    def gather(self, layer: int, slots: torch.Tensor,
               out: tuple[torch.Tensor, torch.Tensor | None] | None = None):
        """(state[layer, slots], conv[layer, slots]) as contiguous [n, ...] buffers."""
        slots = self._check(slots)
        n = slots.numel()
        if out is None:
            st = torch.empty((n, *self.state.shape[2:]), dtype=self.state.dtype, device=self.device)
            cv = (torch.empty((n, *self.conv.shape[2:]), dtype=self.conv.dtype, device=self.device)
                  if self.conv is not None else None)
        else:
            st, cv = out
        self._move("mkv_state_gather", layer, slots, st, cv)
        return st, cv

    def scatter(self, layer: int, slots: torch.Tensor, state: torch.Tensor,
                conv: torch.Tensor | None = None) -> None:
        """state[layer, slots] = state; conv[layer, slots] = conv (unique slots)."""
        slots = self._check(slots, unique=True)
        self._move("mkv_state_scatter", layer, slots, state, conv)

    def _move(self, fn: str, layer: int, slots: torch.Tensor, st: torch.Tensor,
              cv: torch.Tensor | None) -> None:
        n = slots.numel()
        if not 0 <= layer < self.num_layers:
            raise IndexError(f"GDN layer {layer} out of range (pool has {self.num_layers})")
        if st.dtype != self.state.dtype or st.numel() != n * self.state[0, 0].numel():
            raise ValueError("state buffer has the wrong dtype or size")
        if not st.is_contiguous():
            raise ValueError("state buffer must be contiguous")
        use_conv = self.conv is not None and cv is not None
        if use_conv and (cv.dtype != self.conv.dtype or cv.numel() != n * self.conv[0, 0].numel()
                         or not cv.is_contiguous()):
            raise ValueError("conv buffer has the wrong dtype, size or layout")
        _lib.require_gpu(slots, st, self.state, *((cv,) if use_conv else ()))
        if n == 0:
            return
        _lib.call(fn, self.state[layer].data_ptr(), self._entry_bytes(self.state), st.data_ptr(),
                  self.conv[layer].data_ptr() if use_conv else None,
                  self._entry_bytes(self.conv) if use_conv else 0,
                  cv.data_ptr() if use_conv else None, self.num_slots, slots.data_ptr(), n,
                  self._errors.ptr(), _lib.stream_of(self.device))

    def decode_gather(self, layer: int, slots: torch.Tensor, x: torch.Tensor,
                      weight: torch.Tensor, state_out: torch.Tensor | None = None,
                      conv_out: torch.Tensor | None = None):
        """A GDN layer's decode-step state reads in one launch: the batch's
        recurrent states gathered (as ``gather``, without the conv states) and
        the decode conv run in place on the conv slots (as ``conv_decode``).
        Returns (states [B, ...], silu(conv) [B, C])."""
        slots, C, W, w, x, conv_out = self._conv_args(layer, slots, x, weight, conv_out)
        B = slots.numel()
        if state_out is None:
            state_out = torch.empty((B, *self.state.shape[2:]), dtype=self.state.dtype,
                                    device=self.device)
        elif (state_out.dtype != self.state.dtype or not state_out.is_contiguous()
              or state_out.numel() != B * self.state[0, 0].numel()):
            raise ValueError("state_out has the wrong dtype, size or layout")
        _lib.require_gpu(state_out)
        _lib.call("mkv_gdn_decode_gather", self.state[layer].data_ptr(),
                  self._entry_bytes(self.state), state_out.data_ptr(), self.conv[layer].data_ptr(),
                  C, W, self.num_slots, slots.data_ptr(), B, x.data_ptr(), w.data_ptr(),
                  w.shape[1], conv_out.data_ptr(), self._errors.ptr(),
                  _lib.stream_of(self.device))
        return state_out, conv_out

    def _conv_args(self, layer, slots, x, weight, out):
        if self.conv is None:
            raise RuntimeError("this pool keeps no conv states")
        slots = self._check(slots, unique=True)
        if not 0 <= layer < self.num_layers:
            raise IndexError(f"GDN layer {layer} out of range (pool has {self.num_layers})")
        C, W = self.conv.shape[2], self.conv.shape[3]
        B = slots.numel()
        w = weight.reshape(weight.shape[0], -1)
        if x.shape != (B, C) or x.dtype != torch.bfloat16 or self.conv.dtype != torch.bfloat16:
            raise ValueError(f"x must be bf16 [{B}, {C}] and the conv pool bf16")
        if w.shape[0] != C or w.dtype != torch.bfloat16:
            raise ValueError(f"weight must be bf16 [{C}, 1, K]")
        x, w = x.contiguous(), w.contiguous()
        if out is None:
            out = torch.empty_like(x)
        elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError("out must be a contiguous tensor shaped like x")
        _lib.require_gpu(slots, x, w, out, self.conv)
        return slots, C, W, w, x, out

    def conv_decode(self, layer: int, slots: torch.Tensor, x: torch.Tensor,
                    weight: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """The GDN decode conv of one token per request, in place on the conv
        slots (muserve/model/qwen35_layer_v2.py:163-201, decode branch): x
        [B, C] bf16 (one token's mixed_qkv per request), weight [C, 1, 4] or
        [C, 4] bf16 (conv1d.weight) -> silu(conv) [B, C] bf16. Each slot's
        last inputs shift by one with x appended. Slots must be unique. Each
        request has its own state (the reference's decode shares one across
        the batch)."""
        slots, C, W, w, x, out = self._conv_args(layer, slots, x, weight, out)
        B = slots.numel()
        _lib.call("mkv_gdn_conv_decode", self.conv[layer].data_ptr(), self.num_slots, C, W,
                  slots.data_ptr(), B, x.data_ptr(), w.data_ptr(), w.shape[1], out.data_ptr(),
                  self._errors.ptr(), _lib.stream_of(self.device))
        return out

    def check_errors(self) -> None:
        if self._errors is not None:
            self._errors.check("StatePool")
