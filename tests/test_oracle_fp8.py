"""Pins for the fp8 path: torch's e4m3fn cast (the oracle's quantiser) against
hand-derived codes and a brute-force nearest-value search; the kernels' own
encoder/decoder (mkv_common.h, host build) against torch on every fp32 bit
pattern; the quantiser's scale against its closed form."""
import json

import numpy as np
import pytest
import torch

from oracle import fp8 as ref
from tests.helpers import GOLDEN, hostcheck, np_ptr

SPECIAL = json.loads((GOLDEN / "fp8_e4m3fn_special.json").read_text())


def torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn).view(
        torch.uint8).numpy()


def encoder_codes(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.uint8)
    hostcheck().hc_e4m3fn_encode(np_ptr(x), np_ptr(out), x.size)
    return out


def test_special_values_all_agree():
    xs = np.array([e["x"] for e in SPECIAL], np.float32)
    want = np.array([e["code"] for e in SPECIAL], np.uint8)
    assert np.array_equal(torch_codes(xs), want)
    assert np.array_equal(ref.e4m3fn_nearest(xs), want)
    assert np.array_equal(encoder_codes(xs), want)


def structured_floats() -> np.ndarray:
    """Every exponent near the e4m3fn range x every pattern of the top 5
    mantissa bits x low-bit patterns that decide RNE (exact ties, one ulp
    either side, all ones), both signs."""
    exps = np.arange(127 - 14, 127 + 10, dtype=np.uint32)
    top = np.arange(32, dtype=np.uint32) << 18
    low = np.array([0, 1, 2, (1 << 16) - 1, 1 << 16, (1 << 16) + 1, (1 << 17) - 1, 1 << 17,
                    (1 << 17) + 1, (1 << 18) - 1, 12345, 99999], dtype=np.uint32)
    u = (exps[:, None, None] << 23) | top[None, :, None] | low[None, None, :]
    u = u.reshape(-1)
    u = np.concatenate([u, u | np.uint32(0x80000000), np.arange(0, 1 << 12, dtype=np.uint32)])
    return u.view(np.float32)


def test_torch_cast_is_round_to_nearest_even():
    x = structured_floats()
    x = x[np.abs(x.astype(np.float64)) <= 448.0]
    assert x.size > 20000
    assert np.array_equal(torch_codes(x), ref.e4m3fn_nearest(x))


def test_encoder_matches_torch_on_every_fp32_pattern():
    hc = hostcheck()
    chunk = 1 << 24
    for lo in range(0, 1 << 32, chunk):
        u = np.arange(lo, lo + chunk, dtype=np.uint32)
        want = torch.from_numpy(u.view(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8)
        got = np.empty(chunk, np.uint8)
        hc.hc_e4m3fn_encode_bits(lo, lo + chunk, np_ptr(got))
        bad = np.flatnonzero(want.numpy() != got)
        assert bad.size == 0, f"first mismatch at bits {int(u[bad[0]]):#010x}"


def test_decoder_matches_definition_and_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = np.empty(256, np.float32)
    hostcheck().hc_e4m3fn_decode(np_ptr(codes), np_ptr(got), 256)
    tor = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    for c in range(256):
        v = ref.e4m3fn_value(c)
        if np.isnan(v):
            assert np.isnan(got[c]) and np.isnan(tor[c]), c
        else:
            assert got[c] == v == tor[c], c
            assert np.signbit(got[c]) == np.signbit(tor[c]), c


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    u = np.concatenate([
        rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32),
        np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F7FFFFF, 0x00008000,
                  0x3F808000, 0x3F818000, 0x3F807FFF, 0x80000000], dtype=np.uint32)])
    x = u.view(np.float32)
    got = np.empty(x.size, np.uint16)
    hostcheck().hc_bf16_rne(np_ptr(x), np_ptr(got), x.size)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # NaN payloads differ between torch's scalar (0x7FC0) and vector (0xFFFF)
    # CPU paths; any NaN matches any NaN, everything else must be bit-equal.
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    is_bf16_nan = lambda h: ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)
    assert is_bf16_nan(got[nan]).all() and is_bf16_nan(want[nan]).all()


def test_quantize_rows_closed_forms():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 256, generator=g) * 3).bfloat16()
    x[1] = 0                       # all-zero row: scale = float32(1e-12)/448, codes 0
    x[2, 7] = -1e4                 # one big outlier
    q, s = ref.quantize_rows(x)
    amax = x.float().abs().amax(-1)
    want_s = torch.maximum(amax, torch.tensor(1e-12, dtype=torch.float32)) / torch.tensor(
        448.0, dtype=torch.float32)
    assert torch.equal(s, want_s)
    assert s[1].item() == np.float32(np.float32(1e-12) / np.float32(448.0))
    assert (q[1] == 0).all()
    # the element equal to the row absmax lands on +-448 (0x7E / 0xFE)
    i = x.float().abs().argmax(-1)
    top = q[torch.arange(64), i]
    sign = x.float()[torch.arange(64), i] < 0
    nz = amax > 0
    assert torch.equal(top[nz], torch.where(sign, 0xFE, 0x7E).to(torch.uint8)[nz])
    # dequantised values stay within half an fp8 step (1/16 relative) of x
    dq = ref.dequant_rows(q, s).float()
    assert ((dq - x.float()).abs() <= x.float().abs() / 16 + s.unsqueeze(-1) * 2 ** -9).all()


@pytest.mark.parametrize("shape", [(3, 1, 256), (5, 2, 256)])
def test_quantize_rows_is_fast_fp8_quantize_with_row_blocks(shape):
    """block_size = head_dim: per-row blocks of muserve/model/qwen35_layer_v2.py:71-86."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(*shape, generator=g).bfloat16()
    q, s = ref.quantize_rows(x)
    flat = x.reshape(-1, 256).float()
    s2 = flat.abs().amax(-1).clamp(min=1e-12) / 448.0
    q2 = (flat / s2[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(q.reshape(-1, 256), q2) and torch.equal(s.reshape(-1), s2)


def test_reciprocal_divide_equals_division_on_the_quantiser_domain():
    """div_by_recip (mkv_common.h, host build) vs x / scale for every bf16 row
    absmax (hence every reachable scale) and every bf16 x with |x| <= absmax:
    identical e4m3fn codes everywhere, identical quotients where |x/scale| >= 2^-12."""
    import ctypes
    from concurrent.futures import ThreadPoolExecutor

    fn = hostcheck().hc_check_div_by_recip
    fn.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int64

    def run(lo):
        qb, n = ctypes.c_int64(), ctypes.c_int64()
        bad = fn(lo, lo + 0x800, ctypes.addressof(qb), ctypes.addressof(n))
        return bad, qb.value, n.value

    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(run, range(0, 0x8000, 0x800)))
    assert sum(r[0] for r in res) == 0
    assert sum(r[1] for r in res) == 0
    assert sum(r[2] for r in res) == 1073790594
