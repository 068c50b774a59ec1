"""Host tier on the GPU: mkv_pack_blocks / mkv_unpack_blocks vs the oracle
(oracle/state.py pack_blocks / unpack_blocks), with the packed side in device
memory and in pinned host memory; KV pages through the tier; PrefixCache over
device tensors against the reference's OrderedDict model. Byte moves: the bar
is bit-exact."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kv_cache import PagedKVCache
from muserve_amd.memory.host_tier import HostTier
from muserve_amd.model.prefix_cache import PrefixCache
from oracle import state as ref
from oracle.lru import PrefixCacheModel
from oracle.sha import hash_tokens
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


def _pack(pool, ids, out, err):
    planes, P, bb = pool.shape
    _lib.call("mkv_pack_blocks", pool.data_ptr(), P * bb, planes, bb, P, ids.data_ptr(),
              ids.numel(), out.data_ptr(), err.ptr(), _lib.stream_of(DEV))


def _unpack(pool, ids, packed, err):
    planes, P, bb = pool.shape
    _lib.call("mkv_unpack_blocks", pool.data_ptr(), P * bb, planes, bb, P, ids.data_ptr(),
              ids.numel(), packed.data_ptr(), err.ptr(), _lib.stream_of(DEV))


@pytest.mark.parametrize("block_bytes", [16, 64, 8192, 16384, 20000, 3 * 16384 + 48])
@pytest.mark.parametrize("where", ["device", "pinned"])
def test_pack_unpack_match_oracle(block_bytes, where):
    case(f"pack/unpack {block_bytes}-byte blocks, packed side in {where} memory")
    g = torch.Generator().manual_seed(block_bytes)
    planes, P = 3, 37
    pool_cpu = torch.randint(0, 256, (planes, P, block_bytes), generator=g, dtype=torch.uint8)
    pool = pool_cpu.to(DEV)
    ids_cpu = torch.tensor([5, 0, 36, 99, 17, -1, 2], dtype=torch.int32)
    ids = ids_cpu.to(DEV)
    n = ids.numel()
    packed = (torch.full((planes, n, block_bytes), 7, dtype=torch.uint8, device=DEV)
              if where == "device" else
              torch.full((planes, n, block_bytes), 7, dtype=torch.uint8).pin_memory())
    err = _lib.DeviceErrors(DEV)
    _pack(pool, ids, packed, err)
    torch.cuda.synchronize()
    assert torch.equal(packed.cpu(), ref.pack_blocks(pool_cpu, ids_cpu))
    with pytest.raises(_lib.MkvDeviceError, match="state-pool slot out of range"):
        err.check("pack")
    # unpack into a fresh pool: the bad ids are skipped (and flagged)
    back = torch.zeros_like(pool)
    _unpack(back, ids, packed, err)
    torch.cuda.synchronize()
    want = torch.zeros_like(pool_cpu)
    ref.unpack_blocks(want, ids_cpu, packed.cpu())
    assert torch.equal(back.cpu(), want)
    with pytest.raises(_lib.MkvDeviceError):
        err.check("unpack")
    good = [i for i in ids_cpu.tolist() if 0 <= i < P]
    assert torch.equal(back.cpu()[:, good], pool_cpu[:, good])


def _fill(cache, g):
    if cache.dtype == torch.float8_e4m3fn:
        cache.cache.view(torch.uint8).copy_(
            torch.randint(0, 256, cache.cache.shape, generator=g, dtype=torch.uint8))
        cache.scales.copy_(torch.rand(cache.scales.shape, generator=g))
    else:
        cache.cache.copy_(torch.randn(cache.cache.shape, generator=g))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_kv_pages_round_trip_through_the_tier(dtype):
    case(f"host tier KV pages round trip, {dtype}")
    g = torch.Generator().manual_seed(5)
    cache = PagedKVCache(64, num_layers=3, kv_heads=2, dtype=dtype, device=DEV, verbose=False)
    _fill(cache, g)
    before = cache.cache.view(torch.uint8).cpu().clone()
    sbefore = cache.scales.cpu().clone() if cache.scales is not None else None
    src = [3, 17, 40, 41, 9]
    dst = [60, 0, 22, 23, 50]
    tier = HostTier(32 << 20, DEV)
    h = tier.put_blocks(cache.cache, 3, torch.tensor(src))
    hs = tier.put_blocks(cache.scales, 2, torch.tensor(src)) if sbefore is not None else None
    cache.cache.view(torch.uint8).zero_()  # ordered after the pack: the tier holds a copy
    if sbefore is not None:
        cache.scales.zero_()
    tier.get_blocks(h, cache.cache, 3, torch.tensor(dst))
    if hs is not None:
        tier.get_blocks(hs, cache.scales, 2, torch.tensor(dst))
    torch.cuda.synchronize()
    tier.check_errors()
    after = cache.cache.view(torch.uint8).cpu()
    want = torch.zeros_like(before)
    want[:, :, dst] = before[:, :, src]
    assert torch.equal(after, want)
    if sbefore is not None:
        swant = torch.zeros_like(sbefore)
        swant[:, :, dst] = sbefore[:, :, src]
        assert torch.equal(cache.scales.cpu(), swant)
    tier.release(h)
    if hs is not None:
        tier.release(hs)
    assert tier.arena.free_bytes() == tier.arena.nbytes


def test_prefix_cache_device_entries_match_model_and_round_trip():
    case("PrefixCache over device tensors: LRU vs the OrderedDict model, bit-exact restores")
    rng = np.random.default_rng(9)
    g = torch.Generator().manual_seed(9)
    templates = [torch.from_numpy(rng.integers(0, 151936, 64, dtype=np.int64)) for _ in range(5)]
    pc, model = PrefixCache(max_entries=4, host_bytes=16 << 20), PrefixCacheModel(4)
    kept = {}
    for step in range(150):
        t = templates[int(rng.integers(0, 5))]
        ids = torch.cat([t[:int(rng.integers(8, 64))],
                         torch.from_numpy(rng.integers(0, 151936, int(rng.integers(0, 6)),
                                                       dtype=np.int64))])
        if rng.random() < 0.5:
            plen = int(rng.integers(1, len(ids) + 1))
            hidden = torch.randn(plen, 64, generator=g).bfloat16()
            states = [torch.randn(8, 16, 16, generator=g), None, torch.randn(3, 5, generator=g)]
            key = hash_tokens(ids.numpy()[:plen])
            if key not in kept or key not in pc._cache:
                kept[key] = (hidden, states)
            dev_states = [s.to(DEV) if s is not None else None for s in states]
            pc.store(ids.to(DEV), plen, hidden.to(DEV), dev_states)
            for s in dev_states:  # the caller may overwrite its tensors at once
                if s is not None:
                    s.fill_(-1.0)
            model.store(ids.numpy(), plen)
        else:
            hit = pc.lookup(ids, DEV)
            want = model.lookup(ids.numpy())
            assert (hit[0] if hit else None) == want
            if hit:
                h0, s0 = kept[hash_tokens(ids.numpy()[:hit[0]])]
                assert torch.equal(hit[1].cpu(), h0)
                assert hit[2][1] is None
                assert torch.equal(hit[2][0].cpu(), s0[0]) and torch.equal(hit[2][2].cpu(), s0[2])
        assert list(pc._cache) == model.keys()
    pc.sync()
    pc.clear()
    assert pc._tier.arena.free_bytes() == pc._tier.arena.nbytes


def test_prefix_cache_arena_pressure_evicts_lru_first():
    case("PrefixCache arena pressure")
    pc = PrefixCache(max_entries=100, host_bytes=3 << 20)
    base = torch.arange(100, dtype=torch.int64)
    one_mib = torch.zeros(1 << 18, device=DEV)  # 1 MiB of fp32
    for i in range(3):
        pc.store(base + i, 10, one_mib, [])
    assert len(pc) == 3
    pc.lookup(base + 0, DEV)                   # 0 becomes the most recent
    pc.store(base + 3, 10, one_mib, [])        # needs room: 1 (the LRU) leaves
    assert list(pc._cache) == [hash_tokens((base + k).numpy()[:10]) for k in (2, 0, 3)]
    pc.store(base + 4, 10, torch.zeros(1 << 20, device=DEV), [])  # 4 MiB: larger than the arena
    assert len(pc) == 3 and pc.lookup(base + 4, DEV) is None
    pc.sync()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_prefix_cache_keeps_and_restores_kv_pages(dtype):
    case(f"PrefixCache with the prefix's KV pages, {dtype}")
    g = torch.Generator().manual_seed(11)
    cache = PagedKVCache(128, num_layers=4, kv_heads=1, dtype=dtype, device=DEV, verbose=False)
    _fill(cache, g)
    ids = torch.arange(100, dtype=torch.int64)
    prefix_len = 70
    pages = cache.alloc_pages(-(-prefix_len // 16))
    before = cache.cache.view(torch.uint8)[:, :, pages].cpu().clone()
    sbefore = cache.scales[:, :, pages].cpu().clone() if cache.scales is not None else None
    pc = PrefixCache(max_entries=4, host_bytes=64 << 20)
    hidden = torch.randn(prefix_len, 32, generator=g).to(DEV)
    pc.store(ids.to(DEV), prefix_len, hidden, [None], kv=(cache, pages))
    cache.free_pages(pages)
    cache.cache.view(torch.uint8).zero_()  # the pages are reused by others
    hit = pc.lookup_kv(ids, DEV, cache)
    assert hit is not None and hit[0] == prefix_len and len(hit[3]) == len(pages)
    new_pages = hit[3]
    torch.cuda.synchronize()
    pc.sync()
    assert torch.equal(cache.cache.view(torch.uint8)[:, :, new_pages].cpu(), before)
    if sbefore is not None:
        assert torch.equal(cache.scales[:, :, new_pages].cpu(), sbefore)
    assert torch.equal(hit[1].cpu(), hidden.cpu())
