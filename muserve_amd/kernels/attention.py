"""Attention over the KV pool (muserve/kernels/attention.py): paged decode,
and varlen prefill over contiguous K/V or over the pool.

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


def attn_prefill(
    q: torch.Tensor,            # [total_tokens, NUM_Q_HEADS, HEAD_DIM] bf16
    k: torch.Tensor,            # [total_tokens, NUM_KV_HEADS, HEAD_DIM] bf16
    v: torch.Tensor,            # [total_tokens, NUM_KV_HEADS, HEAD_DIM] bf16
    cu_seqlens_q: torch.Tensor, # [num_seqs + 1] int32
    cu_seqlens_k: torch.Tensor, # [num_seqs + 1] int32
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float | None = None,
    causal: bool = True,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:              # [total_tokens, NUM_Q_HEADS, HEAD_DIM] bf16
    """Varlen prefill attention (muserve/kernels/attention.py:6-25, the
    reference's flash_attn_varlen_func): sequence b's queries are rows
    cu_seqlens_q[b]..cu_seqlens_q[b+1] of q, its keys the same rows range of
    cu_seqlens_k in k/v; with causal masking aligned to the bottom-right
    corner (query t of nq sees keys 0 .. nk - nq + t). 4 query heads per KV
    head, head_dim 256; fp32 softmax and accumulation, probabilities rounded
    to bf16 for the P V product, one bf16 rounding of the output."""
    return _prefill(q, k, v, None, cu_seqlens_q, cu_seqlens_k, None, max_seqlen_q, softmax_scale,
                    causal, out, max_seqlen_k)


def attn_prefill_paged(
    q: torch.Tensor,              # [total_tokens, NUM_Q_HEADS, HEAD_DIM] bf16
    k_cache: torch.Tensor,        # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] bf16
    v_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor,   # [num_seqs + 1] int32/int64: the step's query rows
    cache_seqlens: torch.Tensor,  # [num_seqs] int32: keys per sequence, the chunk included
    page_table: torch.Tensor,     # [num_seqs, max_pages] int32
    max_seqlen_q: int,
    softmax_scale: float | None = None,
    causal: bool = True,
    *,
    max_seqlen_k: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """attn_prefill over the paged pool, for chunked prefill: a chunk's
    queries (its K/V appended to the pool first) attend to the sequence's
    cached prefix and to themselves, read through the block table — the
    prefill counterpart of attn_decode. With a scheduler plan, the prefill
    entries are plan.cu_seqlens / plan.seq_lens / plan.block_tables past the
    decode entries. ``max_seqlen_k`` (default: what the table holds) bounds
    cache_seqlens; a tight bound lets short steps split the keys better."""
    if page_table is None:
        raise ValueError("attn_prefill_paged reads the paged pool: page_table is required")
    return _prefill(q, k_cache, v_cache, page_table, cu_seqlens_q, None, cache_seqlens,
                    max_seqlen_q, softmax_scale, causal, out, max_seqlen_k)


PREFILL_Q_TILE = 32            # query tokens per workgroup of the prefill kernel
PREFILL_KV_TILE = 64           # keys per step of the prefill kernel (key ranges are multiples)
PREFILL_SPLIT_MIN = 256        # keys per range at least
_prefill_ws: dict[torch.device, torch.Tensor] = {}
_prefill_min_wg: dict[torch.device, int] = {}


def _prefill_min_workgroups(dev: torch.device) -> int:
    """Below this many query tiles, key ranges are split: one workgroup per
    CU (the kernel's LDS allows one per CU). Measured on MI355X (256 CUs) in
    the serving step, where the prefill attention runs beside the decode
    attention: 256 gave 1.88 ms per step, 320 1.92, 384 1.91, 768 2.00 and
    128 2.17 (more splits leave the decode attention fewer free CUs and
    cost merge traffic; fewer leave CUs idle)."""
    n = _prefill_min_wg.get(dev)
    if n is None:
        n = torch.cuda.get_device_properties(dev).multi_processor_count
        _prefill_min_wg[dev] = n
    return n


def _prefill(q, k, v, page_table, cu_q, cu_k, lens_k, max_seqlen_q, softmax_scale, causal, out,
             max_seqlen_k=None):
    dev = _lib.require_gpu(q, k, v, page_table, cu_q, cu_k, lens_k)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("attn_prefill takes bf16 q, k and v")
    Tq, Hq, D = q.shape
    Hkv = k.shape[-2]
    if D != HEAD_DIM or k.shape[-1] != D or v.shape != k.shape or Hq != 4 * Hkv:
        raise ValueError(f"unsupported shapes q {tuple(q.shape)}, k {tuple(k.shape)} "
                         "(head_dim 256, 4 query heads per KV head)")
    if page_table is not None and (k.dim() != 4 or k.shape[1] != 16):
        raise ValueError("the paged pool must be [num_pages, 16, kv_heads, 256]")
    if page_table is None and k.dim() != 3:
        raise ValueError("contiguous k/v must be [total_tokens, kv_heads, 256]")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("q, k and v must be contiguous")
    cu_q = cu_q.to(device=dev, dtype=torch.int32).contiguous()
    batch = cu_q.numel() - 1
    if cu_k is not None:
        cu_k = cu_k.to(device=dev, dtype=torch.int32).contiguous()
        if cu_k.numel() != batch + 1:
            raise ValueError("cu_seqlens_k must have as many entries as cu_seqlens_q")
    if lens_k is not None:
        if lens_k.dtype != torch.int32 or page_table.dtype != torch.int32:
            raise TypeError("cache_seqlens and page_table must be int32")
        if lens_k.numel() != batch or page_table.shape[0] < batch or page_table.stride(1) != 1:
            raise ValueError("cache_seqlens / page_table rows do not match cu_seqlens_q")
        lens_k = lens_k.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    units = k.shape[0]
    # key-range splits when the query tiles alone would leave most CUs idle
    max_k = int(max_seqlen_k) if max_seqlen_k is not None else page_table.shape[1] * 16
    tiles = -(-int(max_seqlen_q) // PREFILL_Q_TILE) * batch * Hkv
    splits = 1
    min_wg = _prefill_min_workgroups(dev)
    if tiles < min_wg and max_k > PREFILL_SPLIT_MIN:
        splits = min(-(-min_wg // max(tiles, 1)), -(-max_k // PREFILL_SPLIT_MIN))
    split_len = -(-max_k // splits // PREFILL_KV_TILE) * PREFILL_KV_TILE if splits > 1 else 0
    if splits > 1:
        splits = -(-max_k // split_len)
    ws, ws_bytes = None, 0
    if splits > 1:
        ws_bytes = _lib.load().mkv_prefill_attention_workspace_bytes(Tq, Hq, splits)
        ws = _prefill_ws.get(dev)
        if ws is None or ws.numel() < ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            _prefill_ws[dev] = ws
    # the workspace is reused by later calls on the stream: calls on one
    # device must be issued on one stream (or be ordered by the caller)
    _lib.call("mkv_prefill_attention_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), units, Hkv,
              Hq, D, _lib.ptr(page_table), page_table.stride(0) if page_table is not None else 0,
              page_table.shape[1] if page_table is not None else 0, cu_q.data_ptr(),
              _lib.ptr(cu_k), _lib.ptr(lens_k), batch, Tq, int(max_seqlen_q), scale,
              1 if causal else 0, splits, split_len, out.data_ptr(), _lib.ptr(ws), ws_bytes,
              _errword(dev).ptr(), _lib.stream_of(dev))
    return out


def attn_decode(
    q: torch.Tensor,                    # [B, 1, NUM_Q_HEADS, HEAD_DIM] bf16 / fp16
    k_cache: torch.Tensor,              # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] same
    v_cache: torch.Tensor,              # [num_pages, PAGE_SIZE, NUM_KV_HEADS, HEAD_DIM] same
    cache_seqlens: torch.Tensor,        # [B] int32 — current kv length per seq
    page_table: torch.Tensor | None,    # [B, max_pages] int32 — paged kv index
    softmax_scale: float | None = None,
    *,
    max_seqlen: int | None = None,
    out: torch.Tensor | None = None,
    shared_pages: int = 0,
) -> torch.Tensor:                      # [B, 1, NUM_Q_HEADS, HEAD_DIM] bf16 / fp16
    """bf16 or fp16 caches (fp16 is the reference's default pool dtype,
    muserve/config.py:37), with q and the output in the caches' dtype.
    ``max_seqlen`` bounds ``cache_seqlens`` (default: what the page table
    holds). ``out`` may be given to write in place.

    ``shared_pages``: page ids below it may be read by several sequences of
    the batch (prompt pages shared through prefix reuse, e.g. a
    ``BlockManager``'s page range): they are loaded through the GPU caches so
    that their readers share them. Every other page streams past the caches,
    which is faster for pages one sequence reads (the default: 0, no page
    shared).

    With ``page_table=None`` the caches are contiguous per sequence,
    ``[B, S, NUM_KV_HEADS, HEAD_DIM]``, sequence b's first
    ``cache_seqlens[b]`` rows attended (the reference forwards None to its
    kernel the same way, muserve/kernels/attention.py:33-42): the padded
    layout ``PagedKVCache.gather`` writes."""
    fns = {torch.bfloat16: "mkv_decode_attention_bf16", torch.float16: "mkv_decode_attention_f16"}
    if k_cache.dtype not in fns or v_cache.dtype != k_cache.dtype:
        raise TypeError("attn_decode takes bf16 or fp16 caches (attn_decode_fp8 reads fp8 ones)")
    if q.dtype != k_cache.dtype:
        raise TypeError(f"q is {q.dtype}, the caches {k_cache.dtype}: they must match")
    return _decode(fns[k_cache.dtype], q, k_cache, v_cache, None, None, cache_seqlens,
                   page_table, softmax_scale, max_seqlen, out, shared_pages)


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
    shared_pages: int = 0,
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
                   cache_seqlens, page_table, softmax_scale, max_seqlen, out, shared_pages)


def _workspace_for(dev, need):
    ws = _workspace.get(dev)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        _workspace[dev] = ws
    return ws


def _decode_contig(q, k_cache, v_cache, cache_seqlens, softmax_scale, max_seqlen, out):
    dev = _lib.require_gpu(q, k_cache, v_cache, cache_seqlens)
    B, one, Hq, D = q.shape
    if k_cache.dim() != 4:
        raise ValueError("without a page table the caches are [B, S, kv_heads, 256]")
    Bk, S, Hkv, Dk = k_cache.shape
    if one != 1 or D != HEAD_DIM or Dk != D or Bk != B or v_cache.shape != k_cache.shape:
        raise ValueError(f"unsupported shapes q {tuple(q.shape)}, cache {tuple(k_cache.shape)}")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.numel() != B:
        raise TypeError("cache_seqlens must be int32 [B]")
    if not (q.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous()
            and cache_seqlens.is_contiguous()):
        raise ValueError("q, caches and cache_seqlens must be contiguous")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    if max_seqlen is None:
        max_seqlen = S
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    ws = _workspace_for(dev, workspace_bytes(B, Hkv, Hq, max_seqlen))
    _lib.call("mkv_decode_attention_contig", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              1 if k_cache.dtype == torch.float16 else 0, Hkv, Hq, D, S,
              cache_seqlens.data_ptr(), B, int(min(max_seqlen, 1 << 24)), scale, out.data_ptr(),
              ws.data_ptr(), ws.numel(), _errword(dev).ptr(), _lib.stream_of(dev))
    return out


def _decode(fn, q, k_cache, v_cache, k_scales, v_scales, cache_seqlens, page_table,
            softmax_scale, max_seqlen, out, shared_pages=0):
    if page_table is None:
        if k_scales is not None:
            raise ValueError("attn_decode_fp8 reads the paged pool: page_table is required")
        return _decode_contig(q, k_cache, v_cache, cache_seqlens, softmax_scale, max_seqlen, out)
    dev = _lib.require_gpu(q, k_cache, v_cache, k_scales, v_scales, cache_seqlens, page_table)
    B, one, Hq, D = q.shape
    P, page, Hkv, Dk = k_cache.shape
    if one != 1 or page != 16 or D != HEAD_DIM or Dk != D or v_cache.shape != k_cache.shape:
        raise ValueError(f"unsupported shapes q {tuple(q.shape)}, cache {tuple(k_cache.shape)}")
    if q.dtype != (torch.float16 if k_cache.dtype == torch.float16 else torch.bfloat16):
        raise TypeError(f"attn_decode takes a {'fp16' if k_cache.dtype == torch.float16 else 'bf16'}"
                        " query")
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
    ws = _workspace_for(dev, workspace_bytes(B, Hkv, Hq, max_seqlen))
    # the workspace is reused by later calls on the stream: calls on one
    # device must be issued on one stream (or be ordered by the caller)
    scales = () if k_scales is None else (k_scales.data_ptr(), v_scales.data_ptr())
    if shared_pages < 0:
        raise ValueError("shared_pages must be >= 0")
    _lib.call(fn, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), *scales,
              P, int(shared_pages), Hkv, Hq, D, page_table.data_ptr(), page_table.stride(0), width,
              cache_seqlens.data_ptr(), B, max_seqlen, scale, out.data_ptr(),
              ws.data_ptr(), ws.numel(), _errword(dev).ptr(), _lib.stream_of(dev))
    return out
