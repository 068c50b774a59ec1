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


def reset(pool: torch.Tensor, slots) -> None:
    """A new request's states: zeros in every layer of a pool [layers, slots,
    ...] (the torch.zeros of _init_gdn_states / _init_conv_states,
    muserve/model/qwen35_model.py:28-49). Slots outside the pool are skipped."""
    for s in [int(x) for x in slots]:
        if 0 <= s < pool.shape[1]:
            pool[:, s] = 0


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


def conv_decode(conv: torch.Tensor, slots: torch.Tensor, x: torch.Tensor,
                weight: torch.Tensor) -> torch.Tensor:
    """GDN decode conv per request slot (muserve/model/qwen35_layer_v2.py:
    163-201, decode branch :187-192), in float64. conv [slots, C, W] bf16
    holds the last W inputs per channel (W >= K-1; the reference's state is
    [C, K-1]), x [B, C] bf16, weight [C, K] (the conv1d.weight [C, 1, K]).
    Updates conv in place (the shifted state, exact) and returns
    silu(sum_k w[c,k] p_k) [B, C] float64, p = (last K-1 state columns, x).
    Slots outside the pool give zeros and leave the pool unchanged."""
    K = weight.shape[-1]
    W = conv.shape[-1]
    w = weight.reshape(weight.shape[0], K).double()
    out = torch.zeros(x.shape, dtype=torch.float64)
    for b, s in enumerate(slots.tolist()):
        if not 0 <= s < conv.shape[0]:
            continue
        state = conv[s]
        p = torch.cat([state[:, W - (K - 1):].double(), x[b].double().unsqueeze(1)], dim=1)
        acc = (w * p).sum(dim=1)
        out[b] = acc * torch.sigmoid(acc)
        conv[s] = torch.cat([state[:, 1:], x[b].unsqueeze(1).to(state.dtype)], dim=1)
    return out


def conv_decode_reference_fp32(state: torch.Tensor, x: torch.Tensor,
                               weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """_gdn_conv1d_apply's decode branch for one request as the reference
    writes it (muserve/model/qwen35_layer_v2.py:175-199): fp32 F.conv1d over
    [state | x], SiLU, bf16. state [C, K-1] bf16, x [1, C] bf16, weight
    [C, 1, K] bf16 -> (out [1, C] bf16, new state [C, K-1] bf16)."""
    import torch.nn.functional as F
    K = weight.shape[-1]
    C = x.shape[1]
    padded = torch.cat([state.float().unsqueeze(0), x.float().transpose(0, 1).unsqueeze(0)], -1)
    out = F.conv1d(padded, weight.float(), groups=C)
    new_state = padded[0, :, -(K - 1):].to(x.dtype).contiguous()
    out = F.silu(out).squeeze(0).transpose(0, 1).to(x.dtype).contiguous()
    return out, new_state
