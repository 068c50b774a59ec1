"""Paged decode attention (mkv_decode_attention_bf16 through attn_decode) vs
the float64 oracle (oracle/attention.py).

Tolerance: the kernel computes scores, softmax and accumulation in fp32 and
rounds the result to bf16 once, so every output element is within one bf16
ulp of the float64 result (ulp taken at |want|, floor 2^-20 near zero). The
reference's own bf16 path (muserve/model/qwen35_layer_v2.py:493-502) is up to
~2 ulp off the same float64 result (tests/test_oracle_attention.py)."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kernels import attention as A
from oracle import attention as att
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


def build(seed, lens, Hq, Hkv, spare=5, width=None):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    pages = [-(-int(n) // 16) for n in lens]
    P = sum(pages) + spare
    perm = rng.permutation(P)
    W = width or max(1, max(pages))
    table = np.zeros((len(lens), W), dtype=np.int32)
    at = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[at:at + n]
        at += n
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(P, 16, Hkv, 256, generator=g).bfloat16()
    v = torch.randn(P, 16, Hkv, 256, generator=g).bfloat16()
    q = torch.randn(len(lens), 1, Hq, 256, generator=g).bfloat16()
    return q, k, v, lens, table


def within_one_ulp(got: torch.Tensor, want: np.ndarray) -> None:
    got = got.float().cpu().numpy().astype(np.float64)
    mag = np.maximum(np.abs(want), 2.0 ** -13)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
    err = np.abs(got - want)
    bad = err > ulp
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements off by more than 1 bf16 ulp; "
                           f"worst {err[bad].max()} at {np.argwhere(bad)[0]}")


def run(q, k, v, lens, table, max_seqlen=None, scale=None):
    out = A.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV),
                        torch.from_numpy(lens.astype(np.int32)).to(DEV),
                        torch.from_numpy(table).to(DEV), scale, max_seqlen=max_seqlen)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.decode_attention(q[:, 0].float().numpy(), k.float().numpy(), v.float().numpy(),
                                lens, table, 256 ** -0.5 if scale is None else scale)
    return out[:, 0], want


@pytest.mark.parametrize("Hq,Hkv", [(4, 1), (1, 1), (2, 1), (8, 1), (4, 2), (8, 2)])
def test_matches_oracle(Hq, Hkv):
    lens = [1, 2, 15, 16, 17, 31, 33, 200, 511, 512, 513, 1000, 1023, 1024, 1025, 1500, 2049, 3000,
            4097, 0, 7]
    case(f"decode attention Hq={Hq} Hkv={Hkv} lens {lens}")
    q, k, v, lens, table = build(11 + Hq + 10 * Hkv, lens, Hq, Hkv)
    got, want = run(q, k, v, lens, table)
    within_one_ulp(got, want)


def test_tight_bound_and_scale():
    lens = [300, 64, 511, 1]
    case(f"decode attention, max_seqlen 512 (no merge pass), scale 0.1, lens {lens}")
    q, k, v, lens, table = build(21, lens, 4, 1, width=100)
    got, want = run(q, k, v, lens, table, max_seqlen=512, scale=0.1)
    within_one_ulp(got, want)


def test_large_scores_stay_finite():
    # keys aligned with the query: scores in the hundreds, softmax peaked
    lens = [700, 40]
    case("decode attention, large scores")
    q, k, v, lens, table = build(22, lens, 4, 1)
    k = k.float()
    k[table[0, 3], 5, 0] = q[0, 0, 1].float() * 4.0
    k = k.bfloat16()
    got, want = run(q, k, v, lens, table)
    assert torch.isfinite(got.float()).all()
    within_one_ulp(got, want)


def test_bad_page_and_long_sequence_are_flagged():
    case("decode attention, page id past the pool and a length past the table")
    q, k, v, lens, table = build(23, [40, 20], 4, 1)
    table = table.copy()
    table[0, 1] = k.shape[0] + 7  # outside the pool
    lens = lens.copy()
    lens[1] = table.shape[1] * 16 + 5  # longer than the table holds
    A.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(lens.astype(np.int32)).to(DEV),
                  torch.from_numpy(table).to(DEV))
    with pytest.raises(_lib.MkvDeviceError) as e:
        A.check_errors(DEV)
    assert "page id out of range" in str(e.value) and "longer than its block table" in str(e.value)


def test_decode_config_shape_against_oracle():
    # the decode configuration: 256 sequences, lognormal(median 4096, sigma 1)
    # context lengths clipped to 1..32768, 4 query heads over 1 KV head
    rng = np.random.default_rng(102)
    lens = np.clip(np.round(rng.lognormal(np.log(4096.0), 1.0, 256)), 1, 32768).astype(np.int64)
    case(f"decode attention, 256 sequences, {int(lens.sum())} cached tokens")
    q, k, v, lens, table = build(24, lens, 4, 1)
    got, want = run(q, k, v, lens, table, max_seqlen=int(lens.max()))
    within_one_ulp(got, want)
