"""fp8 e4m3fn quantise / dequantise on the CPU (oracle; test infrastructure only).

quantize_rows restates _fast_fp8_quantize of
muserve/model/qwen35_layer_v2.py:71-86 with block_size = the row length, i.e.
one absmax/448 scale per (token, head) row. e4m3fn_nearest and e4m3fn_value
are independent brute-force / definitional restatements of OCP fp8 e4m3fn,
used to pin torch's own cast.
"""
from __future__ import annotations

import numpy as np
import torch


def quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [..., D] -> (q [..., D] uint8 e4m3fn codes, scale [...] fp32).

    qwen35_layer_v2.py:81-85: float upcast, absmax over the block, clamp(min=1e-12),
    /448 (fp32 division), x/scale, clamp to +-448, torch's RNE cast to e4m3fn.
    """
    xf = x.float()
    scale = xf.abs().amax(dim=-1).clamp(min=1e-12) / 448.0
    q = (xf / scale.unsqueeze(-1)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), scale


def dequant_rows(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(float(q) * scale): the inverse scaling, rounded to bf16 (RNE)."""
    return (q.view(torch.float8_e4m3fn).float() * scale.unsqueeze(-1)).to(torch.bfloat16)


def e4m3fn_value(code: int) -> float:
    """Value of an e4m3fn code from the OCP definition (bias 7, no infinities,
    S.1111.111 = NaN, subnormals m * 2^-9)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 0xF and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


_POS_CODES = np.arange(0x7F, dtype=np.int64)                  # 0x00..0x7E, increasing value
_POS_VALUES = np.array([e4m3fn_value(int(c)) for c in _POS_CODES])


def e4m3fn_nearest(x: np.ndarray) -> np.ndarray:
    """Brute-force round-to-nearest-even of float32 values to e4m3fn codes:
    the code whose value is closest to |x| (ties to the even code), with x's
    sign bit; NaN and |x| > 464 (the point past which the nearest value would
    be 480, which e4m3fn lacks) give 0x7F|sign, as torch's cast does."""
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    sign = ((x.view(np.uint32) >> 31).astype(np.uint8)) << 7
    a = np.abs(x.astype(np.float64))
    out = np.empty(x.shape, dtype=np.uint8)
    for lo in range(0, a.size, 1 << 14):
        blk = a[lo:lo + (1 << 14)]
        d = np.abs(blk[:, None] - _POS_VALUES[None, :])
        best = d.argmin(axis=1)
        nxt = np.minimum(best + 1, _POS_VALUES.size - 1)
        tie = (d[np.arange(blk.size), nxt] == d[np.arange(blk.size), best]) & (nxt != best)
        pick = np.where(tie & (best % 2 == 1), nxt, best)
        out[lo:lo + blk.size] = pick
    bad = np.isnan(a) | (a > 464.0)
    out[bad] = 0x7F
    return out | sign
