"""Paged decode attention on the CPU (oracle; test infrastructure only).

muserve's decode attention for one query token per sequence:
  * the paged interface of attn_decode (muserve/kernels/attention.py:29-42):
    q [B,1,Hq,D], k/v cache [P,16,Hkv,D], cache_seqlens [B] int32,
    page_table [B,W] int32 (causal: a decode token sees every cached token);
  * the math of the contiguous decode path (muserve/model/qwen35_layer_v2.py:
    493-502): K/V repeated over the query-head group (repeat_interleave, so
    query head h uses KV head h // G), scores = q k^T * scale, softmax over
    the sequence, weighted sum of V.

`decode_attention` evaluates that in float64 (numpy) from the pages the
table names; `reference_bf16` runs the contiguous path as written, in torch
bf16 on the CPU, on K/V gathered from the same pages.

The reference has no fp8 pool. Over one, the fused decode reads a cached
value as code * scale, taken exactly: `dequant_exact` gives those values
(e4m3fn codes decoded by their OCP definition, fp8.e4m3fn_value) for
`decode_attention` to attend over.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle.fp8 import e4m3fn_value

PAGE = 16
_E4M3FN = np.array([e4m3fn_value(c) for c in range(256)])


def gather_kv(cache: np.ndarray, table_row: np.ndarray, length: int) -> np.ndarray:
    """[P,16,Hkv,D] cache, one sequence's table row -> its first `length`
    tokens as [length, Hkv, D] (muserve/kv_cache.py:149-158 page order)."""
    pages = np.asarray(table_row[: -(-length // PAGE)], dtype=np.int64)
    return cache[pages].reshape(-1, *cache.shape[2:])[:length]


def dequant_exact(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes [..., D] and fp32 scales [...] -> float64
    value(code) * scale [..., D], not rounded (fp8.dequant_rows rounds to bf16)."""
    codes = np.asarray(codes, dtype=np.uint8)
    return _E4M3FN[codes] * np.asarray(scales, dtype=np.float64)[..., None]


def decode_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     seq_lens: np.ndarray, page_table: np.ndarray, scale: float,
                     k_scales: np.ndarray | None = None,
                     v_scales: np.ndarray | None = None, stats: bool = False):
    """q [B,Hq,D], caches [P,16,Hkv,D] (any float dtype; computed in float64),
    seq_lens [B], page_table [B,W] -> [B,Hq,D] float64. Length 0 -> zeros.
    With k_scales / v_scales ([P,16,Hkv] fp32) the caches are uint8 e4m3fn
    codes, read as dequant_exact values. stats=True also returns the attended
    mass sum_j p_j |v_j| / sum_j p_j [B,Hq,D] and max_j |score_j| [B,Hq]
    (what a float evaluation's rounding error scales with)."""
    q = np.asarray(q, dtype=np.float64)
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D))
    mass = np.zeros((B, Hq, D))
    smax = np.zeros((B, Hq))
    for b in range(B):
        n = int(seq_lens[b])
        if n == 0:
            continue
        K = gather_kv(k_cache, page_table[b], n)  # [n, Hkv, D]
        V = gather_kv(v_cache, page_table[b], n)
        if k_scales is not None:
            K = dequant_exact(K, gather_kv(k_scales, page_table[b], n))
            V = dequant_exact(V, gather_kv(v_scales, page_table[b], n))
        K = K.astype(np.float64)
        V = V.astype(np.float64)
        for h in range(Hq):
            s = K[:, h // G] @ q[b, h] * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ V[:, h // G]
            if stats:
                mass[b, h] = (p / p.sum()) @ np.abs(V[:, h // G])
                smax[b, h] = np.abs(s).max()
    return (out, mass, smax) if stats else out


def prefill_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_q, scale: float,
                      causal: bool = True, cu_k=None, lens_k=None, page_table=None,
                      stats: bool = False):
    """Varlen prefill attention in float64: the math of attn_prefill
    (muserve/kernels/attention.py:6-25, flash_attn_varlen_func with causal
    masking aligned to the bottom-right corner, as flash-attention defines it
    for nk != nq), with query head h reading KV head h // G.
    q [Tq,Hq,D]; contiguous k/v [Tk,Hkv,D] with cu_k, or a paged pool
    [P,16,Hkv,D] with page_table [B,W] and lens_k [B]. Sequence b's query
    token t sits at position nk - nq + t and, when causal, attends to
    positions 0..that position; a token that sees nothing gets zeros.
    -> out [Tq,Hq,D] (and, with stats, the attended mass sum p|v| / sum p)."""
    q = np.asarray(q, dtype=np.float64)
    Tq, Hq, D = q.shape
    Hkv = k.shape[-2]
    G = Hq // Hkv
    out = np.zeros((Tq, Hq, D))
    mass = np.zeros((Tq, Hq, D))
    for b in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[b]), int(cu_q[b + 1])
        nq = q1 - q0
        if page_table is not None:
            nk = int(lens_k[b])
            K = gather_kv(k, page_table[b], nk).astype(np.float64)
            V = gather_kv(v, page_table[b], nk).astype(np.float64)
        else:
            k0, k1 = int(cu_k[b]), int(cu_k[b + 1])
            nk = k1 - k0
            K = np.asarray(k[k0:k1], dtype=np.float64)
            V = np.asarray(v[k0:k1], dtype=np.float64)
        for t in range(nq):
            last = nk - nq + t if causal else nk - 1
            if last < 0 or nk == 0:
                continue
            for h in range(Hq):
                s = K[:last + 1, h // G] @ q[q0 + t, h] * scale
                p = np.exp(s - s.max())
                w = p / p.sum()
                out[q0 + t, h] = w @ V[:last + 1, h // G]
                if stats:
                    mass[q0 + t, h] = w @ np.abs(V[:last + 1, h // G])
    return (out, mass) if stats else out


def reference_bf16(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   seq_lens, page_table, scale: float) -> torch.Tensor:
    """muserve/model/qwen35_layer_v2.py:493-502 per sequence, bf16 on the CPU:
    q [B,Hq,D] bf16, caches [P,16,Hkv,D] bf16 -> [B,Hq,D] bf16."""
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    out = torch.zeros(B, Hq, D, dtype=torch.bfloat16)
    for b in range(B):
        n = int(seq_lens[b])
        if n == 0:
            continue
        pages = torch.as_tensor(np.asarray(page_table[b][: -(-n // PAGE)], dtype=np.int64))
        k_full = k_cache[pages].reshape(-1, Hkv, D)[:n].unsqueeze(0)  # [1, S, Hkv, D]
        v_full = v_cache[pages].reshape(-1, Hkv, D)[:n].unsqueeze(0)
        k_exp = k_full.repeat_interleave(G, dim=2)  # [1, S, Hq, D]
        v_exp = v_full.repeat_interleave(G, dim=2)
        q_4d = q[b].unsqueeze(0).unsqueeze(2)  # [1, Hq, 1, D]
        k_4d = k_exp.permute(0, 2, 1, 3)  # [1, Hq, S, D]
        scores = torch.matmul(q_4d, k_4d.transpose(-1, -2).contiguous()) * scale
        weights = torch.softmax(scores, dim=-1)
        v_4d = v_exp.permute(0, 2, 1, 3).contiguous()
        out[b] = torch.matmul(weights, v_4d).squeeze(2)[0]
    return out
