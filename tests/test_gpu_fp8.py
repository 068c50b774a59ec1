"""GPU parity of fp8 e4m3fn quantize-on-append and dequant-gather vs the oracle
(torch-CPU restatement of _fast_fp8_quantize with one block per (token, head))."""
import numpy as np
import pytest
import torch

from muserve_amd.kv_cache import PagedKVCache
from oracle import fp8 as ref
from oracle import paged as pref
from tests.gpu_util import DEV, bits16, case

pytestmark = pytest.mark.gpu


def outlier_kv(g, shape, frac=0.01, scale=20.0):
    x = torch.randn(*shape, generator=g)
    mask = torch.rand(*shape, generator=g) < frac
    return torch.where(mask, x * scale, x).bfloat16()


def special_rows(H):
    rows = torch.zeros(8, H, 256)
    rows[1] = -0.0
    rows[2, :, 5] = 3e38                        # one huge value, rest zero
    rows[3] = torch.linspace(-1e-38, 1e-38, 256)  # bf16 subnormals
    rows[4] = 1.0
    rows[4, :, 0] = -1.0
    rows[5] = torch.arange(256) * 1e-3
    rows[6] = 65504.0
    rows[7, :, ::2] = -7.5
    return rows.bfloat16()


def check_pool(cache, q_cpu, s_cpu):
    got_q = cache.cache.view(torch.uint8).cpu()
    got_s = cache.scales.cpu()
    assert torch.equal(got_q, q_cpu)
    assert torch.equal(got_s.view(torch.int32), s_cpu.view(torch.int32))


@pytest.mark.parametrize("H", [1, 2, 3])  # 1 and 2: specialised kernels; 3: any head count
def test_append_fp8_bit_exact(H):
    case(f"fp8 append H={H}")
    g = torch.Generator().manual_seed(103)
    P, L = 64, 2
    cache = PagedKVCache(P, num_layers=L, kv_heads=H, dtype=torch.float8_e4m3fn, device=DEV,
                         verbose=False)
    T = 300
    slots = torch.randperm(P * 16, generator=g)[:T]
    k = outlier_kv(g, (L, T, H, 256))
    v = outlier_kv(g, (L, T, H, 256))
    k[0, :8], v[1, :8] = special_rows(H), special_rows(H)
    cache.append(slots.to(DEV), k.to(DEV), v.to(DEV))
    q_cpu = torch.zeros(L, 2, P, 16, H, 256, dtype=torch.uint8)
    s_cpu = torch.zeros(L, 2, P, 16, H, dtype=torch.float32)
    for l in range(L):
        for kv, x in ((0, k[l]), (1, v[l])):
            q, s = ref.quantize_rows(x)
            q_cpu[l, kv].view(P * 16, H, 256)[slots] = q
            s_cpu[l, kv].view(P * 16, H)[slots] = s
    check_pool(cache, q_cpu, s_cpu)
    cache.check_errors()


def test_append_fp8_nan_rows_stay_nan():
    case("fp8 append NaN rows")
    cache = PagedKVCache(4, num_layers=1, dtype=torch.float8_e4m3fn, device=DEV, verbose=False)
    x = torch.randn(2, 1, 256).bfloat16()
    x[0, 0, 3] = float("nan")
    cache.append(torch.tensor([0, 1], device=DEV), x.to(DEV), x.to(DEV), layer=0)
    q = cache.cache.view(torch.uint8)[0, 0, 0, :2].cpu()
    assert ((q[0] & 0x7F) == 0x7F).all()            # a NaN scale makes every code NaN
    wq, ws = ref.quantize_rows(x[1])
    assert torch.equal(q[1], wq) and cache.scales[0, 0, 0, 1].cpu().item() == ws.item()
    assert torch.isnan(cache.scales[0, 0, 0, 0]).item()


def test_append_fp8_skip_and_bad_slots():
    case("fp8 append: slot -1 skips, out-of-range slot flagged, 2 heads")
    from muserve_amd import _lib
    g = torch.Generator().manual_seed(5)
    cache = PagedKVCache(4, num_layers=1, kv_heads=2, dtype=torch.float8_e4m3fn, device=DEV,
                         verbose=False)
    x = outlier_kv(g, (3, 2, 256))
    cache.append(torch.tensor([5, -1, 63], device=DEV), x.to(DEV), x.to(DEV), layer=0)
    cache.check_errors()
    q, s = ref.quantize_rows(x)
    pool = cache.cache.view(torch.uint8)[0, 0].reshape(64, 2, 256).cpu()
    scales = cache.scales[0, 0].reshape(64, 2).cpu()
    assert torch.equal(pool[5], q[0]) and torch.equal(pool[63], q[2])
    assert torch.equal(scales[5].view(torch.int32), s[0].view(torch.int32))
    untouched = torch.ones(64, dtype=torch.bool)
    untouched[[5, 63]] = False
    assert pool[untouched].sum().item() == 0 and scales[untouched].abs().sum().item() == 0
    cache.append(torch.tensor([7, 64], device=DEV), x[:2].to(DEV), x[:2].to(DEV), layer=0)
    with pytest.raises(_lib.MkvDeviceError, match="slot_mapping"):
        cache.check_errors()
    assert torch.equal(cache.cache.view(torch.uint8)[0, 1].reshape(64, 2, 256)[7].cpu(), q[0])


def test_chunked_prefill_then_dequant_gather_window():
    """Chunks appended into long contexts, then the last N tokens of every
    request dequant-gathered to bf16 (a scaled-down fp8 chunked-prefill case)."""
    case("fp8 chunked prefill + dequant-gather window")
    g = torch.Generator().manual_seed(103)
    rng = np.random.default_rng(103)
    B, L, chunk, N = 4, 2, 96, 150
    ctx = [300, 417, 96, 130]
    P = sum((c + 15) // 16 for c in ctx) + 8
    cache = PagedKVCache(P, num_layers=L, dtype=torch.float8_e4m3fn, device=DEV, verbose=False)
    pages = rng.permutation(P)
    width = max((c + 15) // 16 for c in ctx)
    bt = torch.zeros(B, width, dtype=torch.int32)
    o = 0
    for b, c in enumerate(ctx):
        n = (c + 15) // 16
        bt[b, :n] = torch.from_numpy(pages[o:o + n].astype(np.int32))
        o += n
    q_cpu = torch.zeros(L, 2, P * 16, 1, 256, dtype=torch.uint8)
    s_cpu = torch.zeros(L, 2, P * 16, 1, dtype=torch.float32)
    done = [0] * B
    while any(d < c for d, c in zip(done, ctx)):
        slots = []
        for b, c in enumerate(ctx):
            n = min(chunk, c - done[b])
            pos = np.arange(done[b], done[b] + n)
            slots.append(bt[b, pos // 16].numpy().astype(np.int64) * 16 + pos % 16)
            done[b] += n
        slots = torch.from_numpy(np.concatenate(slots))
        T = slots.numel()
        k, v = outlier_kv(g, (L, T, 1, 256)), outlier_kv(g, (L, T, 1, 256))
        cache.append(slots.to(DEV), k.to(DEV), v.to(DEV))
        for l in range(L):
            for kv, x in ((0, k[l]), (1, v[l])):
                q, s = ref.quantize_rows(x)
                q_cpu[l, kv, slots], s_cpu[l, kv, slots] = q, s
    check_pool(cache, q_cpu.view(L, 2, P, 16, 1, 256), s_cpu.view(L, 2, P, 16, 1))
    sl = torch.tensor(ctx, dtype=torch.int32)
    starts = torch.clamp(sl - N, min=0)
    kd, vd = cache.gather(None, bt.to(DEV), sl.to(DEV), out_len=N, starts=starts.to(DEV),
                          num_layers=L)
    for l in range(L):
        for kv, got in ((0, kd[l]), (1, vd[l])):
            deq = ref.dequant_rows(q_cpu[l, kv], s_cpu[l, kv])  # [P*16, 1, 256] bf16
            plane = deq.view(P, 16, 1, 256)
            want = pref.gather_padded(plane, bt, sl, N, starts)
            assert torch.equal(bits16(got), want.view(torch.int16)), (l, kv)
    cache.check_errors()


@pytest.mark.parametrize("H", [1, 2])
@pytest.mark.parametrize("packed", [False, True])
def test_dequant_gather_ragged(H, packed):
    """Ragged lengths (0, partial tiles, longer than out_len, unaligned window
    starts) in the padded and the packed layout, one and two heads."""
    case(f"fp8 dequant-gather ragged H={H} packed={packed}")
    from muserve_amd import _lib
    g = torch.Generator().manual_seed(31 + H)
    rng = np.random.default_rng(31 + H)
    P, L = 48, 2
    cache = PagedKVCache(P, num_layers=L, kv_heads=H, dtype=torch.float8_e4m3fn, device=DEV,
                         verbose=False)
    x = outlier_kv(g, (L, P * 16, H, 256))
    cache.append(torch.arange(P * 16, device=DEV), x.to(DEV), outlier_kv(g, x.shape).to(DEV))
    lens = torch.tensor([0, 1, 15, 16, 17, 100, 161, 200], dtype=torch.int32)
    starts = torch.tensor([0, 0, 3, 0, 1, 40, 7, 9], dtype=torch.int32)
    out_len = 150
    W = 13
    bt = torch.from_numpy(rng.integers(0, P, size=(lens.numel(), W)).astype(np.int32))
    win = torch.clamp(torch.minimum(lens - starts, torch.tensor(out_len)), min=0)
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(win.to(torch.int64), 0)])
    kd, vd = cache.gather(None, bt.to(DEV), lens.to(DEV), out_len=out_len, starts=starts.to(DEV),
                          num_layers=L, cu_out=cu.to(DEV) if packed else None)
    cache.check_errors()
    qpool = cache.cache.view(torch.uint8).cpu()
    spool = cache.scales.cpu()
    for l in range(L):
        for kv, got in ((0, kd[l]), (1, vd[l])):
            deq = ref.dequant_rows(qpool[l, kv].reshape(P * 16, H, 256),
                                   spool[l, kv].reshape(P * 16, H))
            want = pref.gather_padded(deq.view(P, 16, H, 256), bt, lens, out_len, starts)
            if packed:
                want = torch.cat([want[b, :int(win[b])] for b in range(lens.numel())])
            assert torch.equal(bits16(got), want.view(torch.int16)), (l, kv)
    bad = bt.clone()
    bad[5, 4] = P + 3  # a page id past the pool: its rows come back as zeros
    kd, _ = cache.gather(0, bad.to(DEV), lens.to(DEV), out_len=out_len, starts=starts.to(DEV))
    with pytest.raises(_lib.MkvDeviceError, match="page id"):
        cache.check_errors()
    rows = torch.arange(out_len) + int(starts[5])
    on_bad = (rows // 16 == 4) & (rows < int(lens[5]))
    assert on_bad.any() and kd[5, on_bad.nonzero().squeeze(1)].cpu().float().abs().sum().item() == 0


def test_hardware_conversions_and_divide_match_cpu_semantics():
    """mkv_check_conversions: v_cvt_pk_fp8_f32 / v_cvt_pk_bf16_f32 on all 2^32
    fp32 patterns, v_cvt_pk_f32_fp8 on all 256 codes, and the quantiser's
    reciprocal divide on its whole domain, all on the device."""
    from muserve_amd import _lib
    case("exhaustive conversion self-test")
    c = _lib.check_conversions(DEV)
    assert c["fp32_values"] == 1 << 32 and c["div_pairs"] == 1073790594, c
    for k in ("fp8_encode_mismatch", "bf16_mismatch", "fp8_decode_mismatch",
              "div_code_mismatch", "div_quotient_mismatch"):
        assert c[k] == 0, c
