"""GPU parity of the paged append / gather / decode-step kernels vs the CPU oracle."""
import json

import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kv_cache import BlockTables, PagedKVCache, SequenceKVState, prefill_slot_mapping
from muserve_amd.memory.kv_cache import KVCache
from oracle import paged as ref
from tests.gpu_util import DEV, bits16, case
from tests.helpers import GOLDEN

pytestmark = pytest.mark.gpu
KNOWN = json.loads((GOLDEN / "reference_known_answers.json").read_text())


def tables(seqs, width=None):
    width = width or max(1, max(len(s.page_table) for s in seqs))
    bt = torch.zeros(len(seqs), width, dtype=torch.int32)
    for b, s in enumerate(seqs):
        bt[b, :len(s.page_table)] = torch.tensor(s.page_table, dtype=torch.int32)
    return bt


def test_write_read_known_answer():
    k = KNOWN["write_read"]
    case("write_kv/get_kv_by_layer exact round trip (default 60-layer fp16 pool)")
    cache = PagedKVCache(num_gpu_pages=k["num_pages"], device=DEV, verbose=False)
    page = cache.alloc_pages(1)[0]
    kk = torch.randn(cache.cache.shape[4], cache.cache.shape[5], device=DEV, dtype=cache.dtype)
    vv = torch.randn(cache.cache.shape[4], cache.cache.shape[5], device=DEV, dtype=cache.dtype)
    cache.write_kv(k["layer"], page, k["slot"], kk, vv)
    torch.cuda.synchronize()
    kc, vc = cache.get_kv_by_layer(k["layer"])
    assert (kc[page, 0] - kk).abs().max().item() == k["max_abs_err"]
    assert (vc[page, 0] - vv).abs().max().item() == k["max_abs_err"]
    cache.check_errors()


def test_write_kv_tensor_indices_match_torch_setitem():
    case("write_kv with page/slot tensors vs torch setitem on CPU")
    cache = PagedKVCache(32, num_layers=3, dtype=torch.bfloat16, device=DEV, verbose=False)
    cpu = torch.zeros_like(cache.cache, device="cpu")
    g = torch.Generator().manual_seed(4)
    pages = torch.randperm(32, generator=g)[:10]
    slots = torch.randint(0, 16, (10,), generator=g)
    k = torch.randn(10, 1, 256, generator=g).bfloat16()
    v = torch.randn(10, 1, 256, generator=g).bfloat16()
    cache.write_kv(2, pages.to(DEV), slots.to(DEV), k.to(DEV), v.to(DEV))
    ref.write_kv(cpu, 2, pages, slots, k, v)
    cache.write_kv(1, 7, slice(3, 6), k[:3], v[:3])
    ref.write_kv(cpu, 1, 7, slice(3, 6), k[:3], v[:3])
    assert torch.equal(bits16(cache.cache), cpu.view(torch.int16))
    cache.check_errors()


def plumbing_case(seed=101):
    g = torch.Generator().manual_seed(seed)
    num_pages, B = 512, 8
    lens = torch.randint(1, 513, (B,), generator=g).tolist()
    cache = PagedKVCache(num_pages, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    cache.shuffle_free_list(g)
    free_before = list(cache._free_pages)
    seqs = [SequenceKVState() for _ in range(B)]
    slots = prefill_slot_mapping(cache, seqs, lens)
    T = sum(lens)
    k = torch.randn(T, 1, 256, generator=g).bfloat16()
    v = torch.randn(T, 1, 256, generator=g).bfloat16()
    return cache, seqs, lens, slots, k, v, free_before


def test_plumbing_config_round_trip():
    """1 layer, 512 pages x 16, 1 KV head of 256, bf16; 8 prompts of
    randint(1,513) tokens on a seeded shuffled free list; append everything,
    gather each sequence back to [len,1,256] and compare bit-exactly."""
    case("plumbing: 8 prompts append + packed and padded gather, seed 101")
    cache, seqs, lens, slots, k, v, free_before = plumbing_case()
    cache.append(slots, k.to(DEV), v.to(DEV), layer=0)
    bt = tables(seqs)
    sl = torch.tensor(lens, dtype=torch.int32)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    kp, vp = cache.gather(0, bt.to(DEV), sl.to(DEV), out_len=max(lens), cu_out=cu.to(DEV))
    assert torch.equal(bits16(kp), k.view(torch.int16))
    assert torch.equal(bits16(vp), v.view(torch.int16))
    W = bt.shape[1] * 16
    kd, vd = cache.gather(0, bt.to(DEV), sl.to(DEV), out_len=W)
    cpu = torch.zeros(1, 2, 512, 16, 1, 256, dtype=torch.bfloat16)
    ref.append(cpu, slots.cpu(), k, v, layer=0)
    assert torch.equal(bits16(kd), ref.gather_padded(cpu[0, 0], bt, sl, W).view(torch.int16))
    assert torch.equal(bits16(vd), ref.gather_padded(cpu[0, 1], bt, sl, W).view(torch.int16))
    assert torch.equal(bits16(cache.cache), cpu.view(torch.int16))
    cache.check_errors()


def test_decode_steps_match_oracle():
    """Batch decode: device slot assignment, all-layer append, padded gather,
    for 40 steps on a 3-layer pool, checked against the oracle every step."""
    rng = np.random.default_rng(102)
    B, L, P = 24, 3, 3000
    ctx = np.clip(np.round(rng.lognormal(np.log(300), 1.0, B)), 1, 1500).astype(int)
    ctx[0], ctx[1] = 16, 15  # page-boundary edge cases
    case(f"decode steps B={B} L={L} P={P}")
    cache = PagedKVCache(P, num_layers=L, dtype=torch.bfloat16, device=DEV, verbose=False)
    g = torch.Generator().manual_seed(102)
    cache.shuffle_free_list(g)
    pool = ref.PoolModel(P, list(cache._free_pages))
    seqs = [SequenceKVState() for _ in range(B)]
    oseqs = [ref.SeqModel() for _ in range(B)]
    slots0 = prefill_slot_mapping(cache, seqs, ctx.tolist())
    oslots0 = [x for s, n in zip(oseqs, ctx) for x in s.add_tokens(pool, int(n))]
    assert slots0.cpu().tolist() == oslots0
    T0 = int(ctx.sum())
    k0 = torch.randn(L, T0, 1, 256, generator=g).bfloat16()
    v0 = torch.randn(L, T0, 1, 256, generator=g).bfloat16()
    cache.append(slots0, k0.to(DEV), v0.to(DEV))
    cpu = torch.zeros(L, 2, P, 16, 1, 256, dtype=torch.bfloat16)
    ref.append(cpu, slots0.cpu(), k0, v0)
    width = (int(ctx.max()) + 60) // 16 + 1
    bt = BlockTables(cache, seqs, max_pages=width)
    for step in range(40):
        slots = bt.decode_step()
        want = ref.decode_step(pool, oseqs)
        assert slots.cpu().tolist() == want, f"step {step}"
        kn = torch.randn(L, B, 1, 256, generator=g).bfloat16()
        vn = torch.randn(L, B, 1, 256, generator=g).bfloat16()
        cache.append(slots, kn.to(DEV), vn.to(DEV))
        ref.append(cpu, torch.tensor(want), kn, vn)
        if step % 13 == 0 or step == 39:
            W = bt.padded_len()
            lens = torch.tensor([s.seq_len for s in oseqs], dtype=torch.int32)
            obt = tables(oseqs, width)
            assert torch.equal(bt.tables.cpu(), obt)
            assert torch.equal(bt.seq_lens.cpu(), lens)
            kd, vd = cache.gather(None, bt.tables, bt.seq_lens, out_len=W, num_layers=L)
            for l in range(L):
                assert torch.equal(bits16(kd[l]), ref.gather_padded(cpu[l, 0], obt, lens, W).view(
                    torch.int16)), f"step {step} layer {l}"
                assert torch.equal(bits16(vd[l]), ref.gather_padded(cpu[l, 1], obt, lens, W).view(
                    torch.int16))
    assert [s.page_table for s in seqs] == [s.page_table for s in oseqs]
    assert torch.equal(bits16(cache.cache), cpu.view(torch.int16))
    cache.check_errors()


@pytest.mark.parametrize("row_heads", [1, 2])
def test_gather_windows_packed_and_empty(row_heads):
    case(f"gather windows/packed/empty, heads={row_heads}")
    rng = np.random.default_rng(7)
    P, B = 200, 9
    cache = PagedKVCache(P, num_layers=2, kv_heads=row_heads, dtype=torch.bfloat16, device=DEV,
                         verbose=False)
    g = torch.Generator().manual_seed(7)
    cpu = torch.randn(cache.cache.shape, generator=g).bfloat16()
    cache.cache.copy_(cpu.to(DEV))
    lens = rng.integers(0, 300, B).astype(np.int32)
    lens[0], lens[1], lens[2] = 0, 1, 16
    width = 20
    bt = torch.from_numpy(np.stack([rng.permutation(P)[:width] for _ in range(B)]).astype(np.int32))
    sl = torch.from_numpy(lens)
    starts = torch.from_numpy(np.maximum(lens - 37, 0).astype(np.int32))
    starts[3] = 5  # unaligned window start
    for layer, out_len, st in [(1, 320, None), (0, 37, starts), (1, 100, starts), (0, 7, None)]:
        kd, vd = cache.gather(layer, bt.to(DEV), sl.to(DEV), out_len=out_len,
                              starts=None if st is None else st.to(DEV))
        assert torch.equal(bits16(kd), ref.gather_padded(cpu[layer, 0], bt, sl, out_len, st).view(
            torch.int16)), (layer, out_len)
        assert torch.equal(bits16(vd), ref.gather_padded(cpu[layer, 1], bt, sl, out_len, st).view(
            torch.int16))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    kp, _ = cache.gather(0, bt.to(DEV), sl.to(DEV), out_len=int(lens.max()), cu_out=cu.to(DEV))
    want = torch.cat(ref.gather_packed(cpu[0, 0], bt, sl))
    assert torch.equal(bits16(kp), want.view(torch.int16))
    # all layers in one launch
    kd, vd = cache.gather(None, bt.to(DEV), sl.to(DEV), out_len=320)
    for l in range(2):
        assert torch.equal(bits16(kd[l]), ref.gather_padded(cpu[l, 0], bt, sl, 320).view(torch.int16))
    cache.check_errors()


def test_device_errors_are_reported_not_faulted():
    case("device error word: bad slot, bad page id, narrow table")
    cache = PagedKVCache(8, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    k = torch.ones(2, 1, 256, dtype=torch.bfloat16, device=DEV)
    cache.append(torch.tensor([3, 8 * 16], device=DEV), k, k, layer=0)  # second slot is past the end
    with pytest.raises(_lib.MkvDeviceError, match="slot_mapping"):
        cache.check_errors()
    assert cache.cache[0, 0, 0, 3].float().sum().item() == 256.0
    cache.append(torch.tensor([-1, 4], device=DEV), k, k, layer=0)  # -1 skips silently
    cache.check_errors()
    bt = torch.tensor([[1, 999]], dtype=torch.int32, device=DEV)
    kd, _ = cache.gather(0, bt, torch.tensor([20], dtype=torch.int32, device=DEV), out_len=32)
    with pytest.raises(_lib.MkvDeviceError, match="page id"):
        cache.check_errors()
    assert kd[0, 16:].float().abs().sum().item() == 0.0  # the bad page's rows are zeros
    kd, _ = cache.gather(0, bt[:, :1], torch.tensor([20], dtype=torch.int32, device=DEV), out_len=32)
    with pytest.raises(_lib.MkvDeviceError, match="block table"):
        cache.check_errors()


@pytest.mark.parametrize("layers,dtype,heads", [(3, torch.float8_e4m3fn, 1), (5, torch.float8_e4m3fn, 1),
                                                (3, torch.bfloat16, 2), (7, torch.bfloat16, 1)])
def test_copy_pages_page_sizes(layers, dtype, heads):
    # 4 KiB (fp8), 8 KiB and 16 KiB pages over odd plane counts, skipped pairs,
    # and the fp8 scale planes (64-byte pages)
    case(f"copy_pages: {layers} layers, {dtype}, {heads} KV heads")
    cache = PagedKVCache(40, num_layers=layers, kv_heads=heads, dtype=dtype, device=DEV,
                         verbose=False)
    g = torch.Generator().manual_seed(layers)
    raw = torch.randint(0, 256, (cache.cache.numel() * cache.cache.element_size(),),
                        generator=g, dtype=torch.uint8)
    cache.cache.view(torch.uint8).view(-1).copy_(raw.to(DEV))
    if cache.scales is not None:
        cache.scales.copy_(torch.rand(cache.scales.shape, generator=g).to(DEV))
    want = cache.cache.view(torch.uint8).cpu().clone()
    want_s = cache.scales.cpu().clone() if cache.scales is not None else None
    src, dst = [1, 5, 9, 30, -1, 12], [2, 6, 0, 31, 7, -1]
    cache.copy_pages(src, dst)
    for s_, d_ in zip(src, dst):
        if s_ >= 0 and d_ >= 0:
            want[:, :, d_] = want[:, :, s_]
            if want_s is not None:
                want_s[:, :, d_] = want_s[:, :, s_]
    assert torch.equal(cache.cache.view(torch.uint8).cpu(), want)
    if want_s is not None:
        assert torch.equal(cache.scales.cpu(), want_s)
    cache.check_errors()


def test_copy_pages_and_kvcache():
    case("copy_pages (copy-on-write) and contiguous KVCache append/get")
    cache = PagedKVCache(16, num_layers=4, dtype=torch.bfloat16, device=DEV, verbose=False)
    g = torch.Generator().manual_seed(9)
    cpu = torch.randn(cache.cache.shape, generator=g).bfloat16()
    cache.cache.copy_(cpu.to(DEV))
    cache.copy_pages([1, 5, 9], [2, 6, 0])
    cpu[:, :, [2, 6, 0]] = cpu[:, :, [1, 5, 9]]
    assert torch.equal(bits16(cache.cache), cpu.view(torch.int16))
    kv = KVCache(64, DEV)
    k = torch.randn(10, 2, 256, generator=g).bfloat16()
    kv.append(7, k.to(DEV), (-k).to(DEV))
    kv.advance(10)
    kv.append(7, k[:3].to(DEV), k[:3].to(DEV))
    kv.advance(3)
    kg, vg = kv.get(7)
    assert torch.equal(bits16(kg), torch.cat([k, k[:3]]).view(torch.int16))
    assert torch.equal(bits16(vg), torch.cat([-k, k[:3]]).view(torch.int16))
    assert kv.cache[0].abs().sum().item() == 0
    cache.check_errors()
