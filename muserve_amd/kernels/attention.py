"""Paged decode attention over the KV pool (muserve/kernels/attention.py).

``attn_decode`` keeps the reference wrapper's signature and meaning
(muserve/kernels/attention.py:29-42): one query token per sequence attends to
its ``cache_seqlens[b]`` cached tokens, found through ``page_table``, with
query head h using KV head h // (Hq / Hkv) — the math of
muserve/model/qwen35_layer_v2.py:493-502, read straight from the pool by a
gfx950 kernel instead of a padded gather plus dense attention. Scores,
softmax and accumulation run in fp32; the output is bf16.

The call is asynchronous on the current stream. Data faults (a page id
outside the pool, a length beyond the table) set bits in a per-device error
word that ``check_errors(device)`` raises.
"""
from __future__ import annotations

import torch

from muserve_amd import _lib

HEAD_DIM = 256
CHUNK = 1024  # tokens per work item of the kernel (sizes the workspace)

_errors: dict[torch.device, _lib.DeviceErrors] = {}
_workspace: dict[torch.device, torch.Tensor] = {}


def _errword(dev: torch.device) -> _lib.DeviceErrors:
    if dev not in _errors:
        _errors[dev] = _lib.DeviceErrors(dev)
    return _errors[dev]


def check_errors(device: torch.device | str = "cuda") -> None:
    """Raises MkvDeviceError for faults flagged by earlier calls (synchronises)."""
    dev = torch.device(device)
    if dev in _errors:
        _errors[dev].check("attn_decode")


def workspace_bytes(batch: int, num_kv_heads: int, num_q_heads: int, max_seqlen: int) -> int:
    n = _lib.load().mkv_decode_attention_workspace_bytes(batch, num_kv_heads, num_q_heads,
                                                         max_seqlen)
    if n < 0:
        raise ValueError("bad attention shape")
    return n


def attn_decode(
    q: torch.Tensor,                    # [B, 1, NUM_Q_HEADS, HEAD_DIM] bf16
    k_cache: torch.Tensor,              # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] bf16
    v_cache: torch.Tensor,              # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] bf16
    cache_seqlens: torch.Tensor,        # [B] int32 — current kv length per seq
    page_table: torch.Tensor | None,    # [B, max_pages] int32 — paged kv index
    softmax_scale: float | None = None,
    *,
    max_seqlen: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:                      # [B, 1, NUM_Q_HEADS, HEAD_DIM] bf16
    """``max_seqlen`` bounds ``cache_seqlens`` (default: what the page table
    holds) and sizes the launch; a tighter bound launches fewer empty
    workgroups. ``out`` may be given to write in place."""
    if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("attn_decode takes bf16 caches (attn_decode_fp8 reads fp8 ones)")
    return _decode("mkv_decode_attention_bf16", q, k_cache, v_cache, None, None, cache_seqlens,
                   page_table, softmax_scale, max_seqlen, out)


def attn_decode_fp8(
    q: torch.Tensor,                    # [B, 1, NUM_Q_HEADS, HEAD_DIM] bf16
    k_cache: torch.Tensor,              # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] e4m3fn
    v_cache: torch.Tensor,              # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] e4m3fn
    k_scales: torch.Tensor,             # [num_pages, PAGE_SIZE, NUM_KV_HEADS] fp32
    v_scales: torch.Tensor,             # [num_pages, PAGE_SIZE, NUM_KV_HEADS] fp32
    cache_seqlens: torch.Tensor,
    page_table: torch.Tensor | None,
    softmax_scale: float | None = None,
    *,
    max_seqlen: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:                      # [B, 1, NUM_Q_HEADS, HEAD_DIM] bf16
    """``attn_decode`` over an fp8 pool (codes plus one fp32 scale per token and
    KV head, as ``PagedKVCache`` appends them), with the dequantisation fused:
    a cached value is ``code * scale`` taken exactly (in fp32), not rounded to
    bf16 first as ``gather``'s dequantisation does. Same arguments otherwise."""
    if k_cache.dtype != torch.float8_e4m3fn or v_cache.dtype != torch.float8_e4m3fn:
        raise TypeError("attn_decode_fp8 takes float8_e4m3fn caches")
    for name, s in (("k_scales", k_scales), ("v_scales", v_scales)):
        if s.dtype != torch.float32 or s.shape != k_cache.shape[:3] or not s.is_contiguous():
            raise ValueError(f"{name} must be contiguous fp32 {tuple(k_cache.shape[:3])}")
    return _decode("mkv_decode_attention_fp8", q, k_cache, v_cache, k_scales, v_scales,
                   cache_seqlens, page_table, softmax_scale, max_seqlen, out)


def _decode(fn, q, k_cache, v_cache, k_scales, v_scales, cache_seqlens, page_table,
            softmax_scale, max_seqlen, out):
    if page_table is None:
        raise ValueError("attn_decode reads the paged pool: page_table is required")
    dev = _lib.require_gpu(q, k_cache, v_cache, k_scales, v_scales, cache_seqlens, page_table)
    B, one, Hq, D = q.shape
    P, page, Hkv, Dk = k_cache.shape
    if one != 1 or page != 16 or D != HEAD_DIM or Dk != D or v_cache.shape != k_cache.shape:
        raise ValueError(f"unsupported shapes q {tuple(q.shape)}, cache {tuple(k_cache.shape)}")
    if q.dtype != torch.bfloat16:
        raise TypeError("attn_decode takes a bf16 query")
    if cache_seqlens.dtype != torch.int32 or page_table.dtype != torch.int32:
        raise TypeError("cache_seqlens and page_table must be int32")
    if not (q.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous()
            and cache_seqlens.is_contiguous() and page_table.stride(1) == 1):
        raise ValueError("q, caches, cache_seqlens and page_table rows must be contiguous")
    width = page_table.shape[1]
    if max_seqlen is None:
        max_seqlen = width * 16
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    need = workspace_bytes(B, Hkv, Hq, max_seqlen)
    ws = _workspace.get(dev)
    if ws is None or ws.numel() < need:
        # zero-filled once: the kernels keep its work counters at zero between calls
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        _workspace[dev] = ws
    # the workspace is reused by later calls on the stream: calls on one
    # device must be issued on one stream (or be ordered by the caller)
    scales = () if k_scales is None else (k_scales.data_ptr(), v_scales.data_ptr())
    _lib.call(fn, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), *scales,
              P, Hkv, Hq, D, page_table.data_ptr(), page_table.stride(0), width,
              cache_seqlens.data_ptr(), B, max_seqlen, scale, out.data_ptr(),
              ws.data_ptr(), ws.numel(), _errword(dev).ptr(), _lib.stream_of(dev))
    return out
