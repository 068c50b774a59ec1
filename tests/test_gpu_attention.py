"""Paged decode attention (mkv_decode_attention_bf16 / _fp8 through attn_decode
/ attn_decode_fp8) vs the float64 oracle (oracle/attention.py). Over an fp8
pool the oracle attends over code * scale taken exactly (dequant_exact).

Tolerance: the kernel computes scores, softmax and accumulation in fp32 and
rounds the result to bf16 once. Each output element is within one bf16 ulp
of the float64 result (ulp taken at |want|) plus the fp32 evaluation error.
That error is bounded by 2^-16 * (1 + max|score|) * A, where A =
sum_j p_j |v_j| / sum_j p_j is the attended mass: 256-term fp32 dot products
give the scores an absolute error of about 2^-16 * (1 + max|score|), which
shifts the weights. The second term matters only where the output cancels to
near zero. The reference's own bf16 path
(muserve/model/qwen35_layer_v2.py:493-502) is up to ~2 ulp off the same
float64 result (tests/test_oracle_attention.py)."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kernels import attention as A
from muserve_amd.kv_cache import PagedKVCache
from oracle import attention as att
from oracle import fp8
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


def within_one_ulp(got: torch.Tensor, want, mant: int = 7, min_exp: int = -126) -> None:
    """want = (out, mass, smax) from att.decode_attention(..., stats=True).
    mant / min_exp: mantissa bits and smallest normal exponent of the output
    type (bf16: 7, -126; fp16: 10, -14, below which its ulp stays 2^-24)."""
    want, mass, smax = want
    got = got.float().cpu().numpy().astype(np.float64)
    mag = np.maximum(np.abs(want), 2.0 ** min_exp)
    tol = 2.0 ** (np.floor(np.log2(mag)) - mant) + 2.0 ** -16 * (1 + smax[..., None]) * mass
    err = np.abs(got - want)
    bad = err > tol
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements off by more than 1 ulp + "
                           f"the fp32 term; worst {err[bad].max()} at {np.argwhere(bad)[0]}")
    # the fp32 term only matters where the output cancels: nearly every element
    # is within one ulp of its own magnitude
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** max(min_exp, -13)))) - mant)
    assert (err <= ulp).mean() > 0.999


def run(q, k, v, lens, table, max_seqlen=None, scale=None):
    out = A.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV),
                        torch.from_numpy(lens.astype(np.int32)).to(DEV),
                        torch.from_numpy(table).to(DEV), scale, max_seqlen=max_seqlen)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.decode_attention(q[:, 0].float().numpy(), k.float().numpy(), v.float().numpy(),
                                lens, table, 256 ** -0.5 if scale is None else scale, stats=True)
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


F16 = dict(mant=10, min_exp=-14)


@pytest.mark.parametrize("Hq,Hkv", [(4, 1), (1, 1), (8, 2)])
def test_f16_matches_oracle(Hq, Hkv):
    """fp16 pools (the reference's default KV dtype, muserve/config.py:37):
    q, caches and output fp16; one fp16 ulp of float64 plus the fp32 term."""
    lens = [1, 16, 17, 33, 511, 1024, 1025, 2049, 0, 3000]
    case(f"decode attention fp16 Hq={Hq} Hkv={Hkv} lens {lens}")
    q, k, v, lens, table = build(61 + Hq + 10 * Hkv, lens, Hq, Hkv)
    q, k, v = q.half(), k.half(), v.half()
    got, want = run(q, k, v, lens, table)
    assert got.dtype == torch.float16
    within_one_ulp(got, want, **F16)


def test_f16_reads_the_default_pool():
    """PagedKVCache() with the reference's default dtype (fp16): append, then
    attn_decode over the pool's layer views against the oracle."""
    rng = np.random.default_rng(62)
    lens = rng.integers(1, 1500, 12)
    case(f"default fp16 pool append then decode attention, lens {lens.tolist()}")
    cache = PagedKVCache(int(sum(-(-int(n) // 16) for n in lens)) + 4, num_layers=2, device=DEV,
                         verbose=False)
    assert cache.dtype == torch.float16
    from muserve_amd.kv_cache import SequenceKVState, prefill_slot_mapping
    seqs = [SequenceKVState() for _ in lens]
    slots = prefill_slot_mapping(cache, seqs, [int(n) for n in lens])
    g = torch.Generator().manual_seed(62)
    T = int(lens.sum())
    kv = torch.randn(T, 1, 256, generator=g).half()
    cache.append(slots, kv.to(DEV), (-kv).to(DEV), layer=1)
    table = np.zeros((len(lens), max(len(s.page_table) for s in seqs)), dtype=np.int32)
    for b, s in enumerate(seqs):
        table[b, :len(s.page_table)] = s.page_table
    q = torch.randn(len(lens), 1, 4, 256, generator=g).half()
    out = A.attn_decode(q.to(DEV), *cache.get_kv_by_layer(1),
                        torch.from_numpy(lens.astype(np.int32)).to(DEV),
                        torch.from_numpy(table).to(DEV))
    torch.cuda.synchronize()
    cache.check_errors()
    A.check_errors(DEV)
    kc, vc = cache.get_kv_by_layer(1)
    want = att.decode_attention(q[:, 0].float().numpy(), kc.float().cpu().numpy(),
                                vc.float().cpu().numpy(), lens, table, 256 ** -0.5, stats=True)
    within_one_ulp(out[:, 0], want, **F16)


def test_dtype_mismatch_is_rejected():
    case("attn_decode with a bf16 query over fp16 caches (rejected on the host)")
    q = torch.zeros(1, 1, 4, 256, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(2, 16, 1, 256, dtype=torch.float16, device=DEV)
    with pytest.raises(TypeError, match="must match"):
        A.attn_decode(q, kc, kc, torch.ones(1, dtype=torch.int32, device=DEV),
                      torch.zeros(1, 1, dtype=torch.int32, device=DEV))


def test_decode_config_shape_against_oracle():
    # the decode configuration: 256 sequences, lognormal(median 4096, sigma 1)
    # context lengths clipped to 1..32768, 4 query heads over 1 KV head
    rng = np.random.default_rng(102)
    lens = np.clip(np.round(rng.lognormal(np.log(4096.0), 1.0, 256)), 1, 32768).astype(np.int64)
    case(f"decode attention, 256 sequences, {int(lens.sum())} cached tokens")
    q, k, v, lens, table = build(24, lens, 4, 1)
    got, want = run(q, k, v, lens, table, max_seqlen=int(lens.max()))
    within_one_ulp(got, want)


# ---- fp8 pools: the dequantisation fused into the kernel ----

def quantize(k, v):
    kc, ks = fp8.quantize_rows(k)  # uint8 codes, fp32 per-row scales
    vc, vs = fp8.quantize_rows(v)
    return kc, ks, vc, vs


def run_fp8(q, kc, ks, vc, vs, lens, table, max_seqlen=None, scale=None):
    f8 = torch.float8_e4m3fn
    out = A.attn_decode_fp8(q.to(DEV), kc.view(f8).to(DEV), vc.view(f8).to(DEV), ks.to(DEV),
                            vs.to(DEV), torch.from_numpy(lens.astype(np.int32)).to(DEV),
                            torch.from_numpy(table).to(DEV), scale, max_seqlen=max_seqlen)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.decode_attention(q[:, 0].float().numpy(), kc.numpy(), vc.numpy(), lens, table,
                                256 ** -0.5 if scale is None else scale, ks.numpy(), vs.numpy(),
                                stats=True)
    return out[:, 0], want


@pytest.mark.parametrize("Hq,Hkv", [(4, 1), (1, 1), (2, 1), (8, 1), (8, 2)])
def test_fp8_matches_oracle(Hq, Hkv):
    lens = [1, 2, 15, 16, 17, 33, 511, 512, 513, 1023, 1024, 1025, 2049, 4097, 0, 7]
    case(f"fp8 decode attention Hq={Hq} Hkv={Hkv} lens {lens}")
    q, k, v, lens, table = build(31 + Hq + 10 * Hkv, lens, Hq, Hkv)
    got, want = run_fp8(q, *quantize(k, v), lens, table)
    within_one_ulp(got, want)


def test_fp8_wide_scales_and_outliers():
    # rows scaled by 2^-10 .. 2^10 and 1 % outliers: per-token scales far apart,
    # codes down to the subnormals
    lens = [700, 1500, 64]
    case(f"fp8 decode attention, scales over 2^+-10 and outliers, lens {lens}")
    q, k, v, lens, table = build(32, lens, 4, 1)
    g = torch.Generator().manual_seed(32)
    row = 2.0 ** (torch.rand(*k.shape[:3], 1, generator=g) * 20 - 10)
    out_k = torch.where(torch.rand(k.shape, generator=g) < 0.01, 20.0, 1.0)
    k = (k.float() * row * out_k / 64).bfloat16()  # scores of order one
    v = (v.float() * row.flip(0) * out_k.flip(1)).bfloat16()
    kc, ks, vc, vs = quantize(k, v)
    assert ((kc & 0x78) == 0).any() and ((vc & 0x78) == 0).any()  # subnormal codes present
    got, want = run_fp8(q, kc, ks, vc, vs, lens, table, scale=0.3)
    within_one_ulp(got, want)


def test_fp8_every_code():
    # codes drawn uniformly from all 254 non-NaN values (subnormals, -0 and
    # +-448 included) with random positive scales
    lens = [1000, 333, 2048]
    case(f"fp8 decode attention, uniform codes, lens {lens}")
    q, k, v, lens, table = build(33, lens, 4, 1)
    rng = np.random.default_rng(33)
    allowed = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    kc = torch.from_numpy(rng.choice(allowed, size=k.shape))
    vc = torch.from_numpy(rng.choice(allowed, size=v.shape))
    ks = torch.from_numpy(rng.uniform(0.1, 1.0, k.shape[:3]).astype(np.float32) / 500)
    vs = torch.from_numpy(rng.uniform(0.1, 1.0, v.shape[:3]).astype(np.float32))
    got, want = run_fp8(q, kc, ks, vc, vs, lens, table)
    within_one_ulp(got, want)


def test_fp8_reads_what_the_pool_appends():
    # PagedKVCache(fp8).append quantises on the way in; attention then reads
    # the pool's own codes and scale planes for layer 1
    lens = np.array([37, 1040, 16, 500], dtype=np.int64)
    case(f"fp8 pool append then decode attention, lens {lens.tolist()}")
    q, k, v, lens, table = build(34, lens, 4, 1, spare=9)
    P = k.shape[0]
    cache = PagedKVCache(num_layers=2, num_gpu_pages=P, kv_heads=1, dtype=torch.float8_e4m3fn,
                         device=DEV, verbose=False)
    slots = np.concatenate([table[b, np.arange(n) // 16].astype(np.int64) * 16 + np.arange(n) % 16
                            for b, n in enumerate(lens)])
    kt = torch.cat([torch.from_numpy(att.gather_kv(k.float().numpy(), table[b], int(n)))
                    for b, n in enumerate(lens)]).bfloat16()
    vt = torch.cat([torch.from_numpy(att.gather_kv(v.float().numpy(), table[b], int(n)))
                    for b, n in enumerate(lens)]).bfloat16()
    cache.append(torch.from_numpy(slots).to(DEV), kt.to(DEV), vt.to(DEV), layer=1)
    out = A.attn_decode_fp8(q.to(DEV), cache.cache[1, 0], cache.cache[1, 1], cache.scales[1, 0],
                            cache.scales[1, 1], torch.from_numpy(lens.astype(np.int32)).to(DEV),
                            torch.from_numpy(table).to(DEV))
    torch.cuda.synchronize()
    A.check_errors(DEV)
    cache.check_errors()
    # the oracle quantises the same tokens on the CPU
    kc, ks, vc, vs = (torch.zeros(P, 16, 1, 256, dtype=torch.uint8), torch.zeros(P, 16, 1),
                      torch.zeros(P, 16, 1, 256, dtype=torch.uint8), torch.zeros(P, 16, 1))
    qk, sk = fp8.quantize_rows(kt)
    qv, sv = fp8.quantize_rows(vt)
    sl = torch.from_numpy(slots)
    kc.view(-1, 1, 256)[sl], ks.view(-1, 1)[sl] = qk, sk
    vc.view(-1, 1, 256)[sl], vs.view(-1, 1)[sl] = qv, sv
    want = att.decode_attention(q[:, 0].float().numpy(), kc.numpy(), vc.numpy(), lens, table,
                                256 ** -0.5, ks.numpy(), vs.numpy(), stats=True)
    within_one_ulp(out[:, 0], want)


def test_fp8_bad_page_is_flagged():
    case("fp8 decode attention, page id past the pool")
    q, k, v, lens, table = build(35, [40, 20], 4, 1)
    kc, ks, vc, vs = quantize(k, v)
    table = table.copy()
    table[1, 0] = -3
    f8 = torch.float8_e4m3fn
    A.attn_decode_fp8(q.to(DEV), kc.view(f8).to(DEV), vc.view(f8).to(DEV), ks.to(DEV), vs.to(DEV),
                      torch.from_numpy(lens.astype(np.int32)).to(DEV),
                      torch.from_numpy(table).to(DEV))
    with pytest.raises(_lib.MkvDeviceError) as e:
        A.check_errors(DEV)
    assert "page id out of range" in str(e.value)


def test_fp8_decode_config_shape_against_oracle():
    # 256 sequences, lognormal(median 4096, sigma 1) lengths clipped to 1..32768
    rng = np.random.default_rng(103)
    lens = np.clip(np.round(rng.lognormal(np.log(4096.0), 1.0, 256)), 1, 32768).astype(np.int64)
    case(f"fp8 decode attention, 256 sequences, {int(lens.sum())} cached tokens")
    q, k, v, lens, table = build(36, lens, 4, 1)
    got, want = run_fp8(q, *quantize(k, v), lens, table, max_seqlen=int(lens.max()))
    within_one_ulp(got, want)


@pytest.mark.parametrize("batch,Hkv", [(4096, 1), (1500, 2), (300, 1)])
def test_work_list_sizes(batch, Hkv):
    # the chunk kernel's work list (one entry per sequence and KV head, up to
    # 4096, in LDS) at its largest, at more than one round of its 256-pair
    # passes and at one round, over bf16 and fp8 pools
    rng = np.random.default_rng(37 + batch)
    lens = rng.integers(0, 1200, batch)
    lens[::97] = 2048 + rng.integers(0, 2048, len(lens[::97]))  # some two- and three-chunk pairs
    case(f"decode attention work list: batch {batch} x {Hkv} KV heads, {int(lens.sum())} tokens")
    q, k, v, lens, table = build(38 + batch, lens, 4 * Hkv, Hkv)
    got, want = run(q, k, v, lens, table)
    within_one_ulp(got, want)
    got, want = run_fp8(q, *quantize(k, v), lens, table)
    within_one_ulp(got, want)


# ---- contiguous caches: attn_decode with page_table=None ----

def contiguous_from_pages(x, lens, table, S, pad_value):
    """[B, S, Hkv, 256] per-sequence rows from a paged pool; rows past a
    sequence's length hold pad_value."""
    B = len(lens)
    out = torch.full((B, S) + tuple(x.shape[2:]), pad_value, dtype=x.dtype)
    for b, n in enumerate(lens):
        out[b, :n] = torch.from_numpy(att.gather_kv(x.float().numpy(), table[b], int(n))).to(x.dtype)
    return out


@pytest.mark.parametrize("Hq,Hkv,dtype", [(4, 1, torch.bfloat16), (8, 2, torch.bfloat16),
                                          (4, 1, torch.float16)])
def test_contiguous_caches_match_oracle(Hq, Hkv, dtype):
    """page_table=None: caches [B, S, Hkv, 256] (S = 1000, not a multiple of
    16, the last sequence using every row); rows past each length hold NaN,
    which must not reach the output."""
    lens = [1, 16, 17, 999, 0, 513, 1000]
    case(f"decode attention over contiguous caches Hq={Hq} Hkv={Hkv} {dtype} lens {lens}")
    q, k, v, lens, table = build(81 + Hq, lens, Hq, Hkv)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    S = 1000
    kc = contiguous_from_pages(k, lens, table, S, float("nan"))
    vc = contiguous_from_pages(v, lens, table, S, float("nan"))
    out = A.attn_decode(q.to(DEV), kc.to(DEV), vc.to(DEV),
                        torch.from_numpy(lens.astype(np.int32)).to(DEV), None)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.decode_attention(q[:, 0].float().numpy(), k.float().numpy(), v.float().numpy(),
                                lens, table, 256 ** -0.5, stats=True)
    assert torch.isfinite(out.float()).all()
    within_one_ulp(out[:, 0], want, **(F16 if dtype == torch.float16 else {}))


def test_contiguous_equals_paged_on_the_gathered_layout():
    """The padded gather's output [B, Lpad, 1, 256] read with page_table=None
    gives the same bits as attention over the pool it was gathered from (the
    same pages per sequence, so the same work split and summation order)."""
    rng = np.random.default_rng(82)
    lens = rng.integers(1, 3000, 40)
    case(f"gather then contiguous decode attention vs paged, lens sum {int(lens.sum())}")
    q, k, v, lens, table = build(82, lens, 4, 1)
    cache = PagedKVCache(k.shape[0], num_layers=1, dtype=torch.bfloat16, device=DEV,
                         verbose=False)
    cache.cache[0, 0].copy_(k.to(DEV))
    cache.cache[0, 1].copy_(v.to(DEV))
    lt = torch.from_numpy(lens.astype(np.int32)).to(DEV)
    tt = torch.from_numpy(table).to(DEV)
    out_len = table.shape[1] * 16
    kg, vg = cache.gather(0, tt, lt, out_len=out_len)
    paged = A.attn_decode(q.to(DEV), *cache.get_kv_by_layer(0), lt, tt)
    contig = A.attn_decode(q.to(DEV), kg, vg, lt, None)
    torch.cuda.synchronize()
    cache.check_errors()
    A.check_errors(DEV)
    assert torch.equal(paged.view(torch.int16), contig.view(torch.int16))


def test_contiguous_length_past_the_rows_is_flagged():
    case("decode attention over contiguous caches, a length past the rows")
    q = torch.randn(2, 1, 4, 256).bfloat16().to(DEV)
    kc = torch.randn(2, 40, 1, 256).bfloat16().to(DEV)
    A.attn_decode(q, kc, kc, torch.tensor([40, 41], dtype=torch.int32, device=DEV), None)
    with pytest.raises(_lib.MkvDeviceError, match="longer than its block table"):
        A.check_errors(DEV)


@pytest.mark.parametrize("Hq,Hkv,lens", [
    (4, 1, [1, 2, 15, 16, 17, 31, 33, 200, 511, 512, 513, 1000, 1023, 1024, 1025, 1500, 2049, 3000,
            4097, 0, 7]),
    (8, 2, [1, 17, 513, 2049, 0, 3000, 64]),
    (1, 1, [30000]),                    # one sequence over many waves
    (4, 1, [16] * 1500 + [300, 0, 5]),  # more sequences than half the waves: unaligned spans
    (4, 1, [0] * 1000 + [700] * 90 + [3, 17]),  # aligned spans, too many pairs to sort
])
def test_shared_pages_shapes(Hq, Hkv, lens):
    """The shared-page variant (every page below the bound through the
    caches; each sequence's pages start a wave's span while the sequences
    number at most half the waves, in the order of their first page id up to
    1024 pairs) against the oracle."""
    case(f"decode attention, shared_pages = pool, Hq={Hq} Hkv={Hkv}, {len(lens)} sequences, "
         f"max {max(lens)}")
    q, k, v, lens, table = build(95 + Hq + 10 * Hkv, lens, Hq, Hkv)
    out = A.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV),
                        torch.from_numpy(lens.astype(np.int32)).to(DEV),
                        torch.from_numpy(table).to(DEV), shared_pages=k.shape[0])
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.decode_attention(q[:, 0].float().numpy(), k.float().numpy(), v.float().numpy(),
                                lens, table, 256 ** -0.5, stats=True)
    within_one_ulp(out[:, 0], want)


@pytest.mark.parametrize("fp8", [False, True])
def test_shared_pages_bound(fp8):
    """shared_pages (pages below it loaded through the caches, the rest
    streamed past them; every sequence's pages start a wave's span) against
    the oracle, with sequences sharing a common prefix of pages as prefix
    reuse makes them. Bounds 16, P/2 and P give the same bits: they change
    only which loads go through the caches."""
    rng = np.random.default_rng(91)
    lens = rng.integers(300, 2500, 48)
    lens[5] = 0  # an empty sequence among them
    case(f"decode attention, shared prefix pages, shared_pages bound, fp8={fp8}")
    q, k, v, lens, table = build(91, lens, 4, 1, spare=40)
    table = table.copy()
    table[::3, :16] = np.arange(16, dtype=np.int32)  # a third share the pool's first 16 pages
    lt = torch.from_numpy(lens.astype(np.int32)).to(DEV)
    tt = torch.from_numpy(table).to(DEV)
    P = k.shape[0]
    if fp8:
        kc, ks, vc, vs = quantize(k, v)
        f8 = torch.float8_e4m3fn
        args = (q.to(DEV), kc.view(f8).to(DEV), vc.view(f8).to(DEV), ks.to(DEV), vs.to(DEV), lt, tt)
        fn = A.attn_decode_fp8
        want = att.decode_attention(q[:, 0].float().numpy(), kc.numpy(), vc.numpy(), lens, table,
                                    256 ** -0.5, ks.numpy(), vs.numpy(), stats=True)
    else:
        args = (q.to(DEV), k.to(DEV), v.to(DEV), lt, tt)
        fn = A.attn_decode
        want = att.decode_attention(q[:, 0].float().numpy(), k.float().numpy(),
                                    v.float().numpy(), lens, table, 256 ** -0.5, stats=True)
    first = None
    for bound in (16, P // 2, P):
        got = fn(*args, shared_pages=bound)
        torch.cuda.synchronize()
        A.check_errors(DEV)
        within_one_ulp(got[:, 0], want)
        if first is None:
            first = got
        assert torch.equal(got.view(torch.int16), first.view(torch.int16)), bound


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_against_oracle(seed):
    """Seeded sweep: pool kind (bf16 / fp16 / fp8), query heads per KV head,
    one or two KV heads, batch size, lengths (empty, one token, page
    boundaries, long), sequences sharing leading pages, and shared_pages off
    or covering the pool; each case against the float64 oracle."""
    rng = np.random.default_rng(1000 + seed)
    kind = ("bf16", "f16", "fp8")[seed % 3]
    Hkv = 2 if seed % 4 == 3 and kind != "fp8" else 1
    G = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 64))
    lens = rng.integers(0, 3000, B)
    special = [0, 1, 15, 16, 17, 4096 + 3]
    for i in range(min(B, 3)):
        lens[int(rng.integers(0, B))] = special[int(rng.integers(0, len(special)))]
    q, k, v, lens, table = build(2000 + seed, lens, G * Hkv, Hkv, spare=24)
    if B > 2 and rng.random() < 0.7:  # some sequences share leading pages
        table = table.copy()
        share = int(rng.integers(1, 24))
        for b in range(B):
            if rng.random() < 0.5 and lens[b] > 16 * share:
                table[b, :share] = table[0, :share] if lens[0] > 16 * share else np.arange(share)
    shared = int(k.shape[0]) if seed % 2 else 0
    case(f"decode attention sweep seed {seed}: {kind}, G={G}, Hkv={Hkv}, B={B}, "
         f"max len {int(lens.max())}, shared_pages {shared}")
    lt = torch.from_numpy(lens.astype(np.int32)).to(DEV)
    tt = torch.from_numpy(table).to(DEV)
    if kind == "fp8":
        kc, ks, vc, vs = quantize(k, v)
        f8 = torch.float8_e4m3fn
        got = A.attn_decode_fp8(q.to(DEV), kc.view(f8).to(DEV), vc.view(f8).to(DEV), ks.to(DEV),
                                vs.to(DEV), lt, tt, shared_pages=shared)
        want = att.decode_attention(q[:, 0].float().numpy(), kc.numpy(), vc.numpy(), lens, table,
                                    256 ** -0.5, ks.numpy(), vs.numpy(), stats=True)
        tol = {}
    else:
        dt = torch.bfloat16 if kind == "bf16" else torch.float16
        q, k, v = q.to(dt), k.to(dt), v.to(dt)
        got = A.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV), lt, tt, shared_pages=shared)
        want = att.decode_attention(q[:, 0].float().numpy(), k.float().numpy(),
                                    v.float().numpy(), lens, table, 256 ** -0.5, stats=True)
        tol = F16 if kind == "f16" else {}
    torch.cuda.synchronize()
    A.check_errors(DEV)
    within_one_ulp(got[:, 0], want, **tol)
