"""Host bookkeeping of the paged pool vs the reference's known answers and the
oracle (no GPU: the pool lives on the CPU and only metadata calls run)."""
import json

import numpy as np
import pytest
import torch

from muserve_amd.kv_cache import (PagedKVCache, SequenceKVState, prefill_slot_mapping,
                                  slot_mapping_for)
from muserve_amd.memory.kv_cache import KVCache
from oracle import paged as ref
from tests.helpers import GOLDEN

KNOWN = json.loads((GOLDEN / "reference_known_answers.json").read_text())


def cpu_cache(n, **kw):
    return PagedKVCache(n, num_layers=1, device="cpu", verbose=False, **kw)


@pytest.mark.parametrize("impl", ["product", "oracle"])
def test_alloc_free_known_answers(impl):
    k = KNOWN["alloc_free"]
    if impl == "product":
        c = cpu_cache(k["num_pages"])
        alloc, free, count = c.alloc_pages, c.free_pages, lambda: c.num_free_pages
    else:
        m = ref.PoolModel(k["num_pages"])
        alloc, free, count = m.alloc, m.release, lambda: m.num_free
    last = None
    for st in k["steps"]:
        if st["op"] == "alloc":
            last = alloc(st["n"])
            assert len(last) == st["returned"] and count() == st["free_after"]
        elif st["op"] == "free_first_of_last_alloc":
            free(last[:st["n"]])
            assert count() == st["free_after"]
        else:
            before = count()
            with pytest.raises(RuntimeError, match="KV cache OOM"):
                alloc(st["n"])
            assert count() == before  # nothing changed


def test_alloc_order_matches_oracle_lifo():
    rng = np.random.default_rng(7)
    c, m = cpu_cache(300), ref.PoolModel(300)
    for _ in range(200):
        if rng.random() < 0.6 and m.num_free:
            n = int(rng.integers(1, min(m.num_free, 20) + 1))
            assert c.alloc_pages(n) == m.alloc(n)
        else:
            taken = [p for p in range(300) if p not in set(m.free)]
            back = list(rng.permutation(taken)[:int(rng.integers(0, 6))].tolist())
            c.free_pages(back)
            m.release(back)
        assert c._free_pages == m.free and c.num_free_pages == m.num_free
    assert c.num_free_tokens() == 16 * c.num_free_pages


def test_alloc_zero_takes_whole_list_like_reference():
    # muserve/kv_cache.py:84-86 with n == 0: free[-0:] is the whole list
    c, m = cpu_cache(8), ref.PoolModel(8)
    assert c.alloc_pages(0) == m.alloc(0) == list(range(8))
    assert c._free_pages == m.free == [] and c.num_free_pages == m.num_free == 8


def test_sequence_state_known_answers():
    k = KNOWN["sequence_state"]
    c = cpu_cache(k["num_pages"])
    seq = SequenceKVState()
    for _ in range(k["tokens"]):
        if seq.needs_new_page():
            seq.page_table.append(c.alloc_pages(1)[0])
        seq.seq_len += 1
    assert seq.num_pages_used == k["pages_used"] and seq.seq_len == k["seq_len"]
    assert seq.last_page_slot == k["last_page_slot"]
    pt = seq.to_page_table_tensor(max_pages=k["table_width"], device="cpu")
    assert tuple(pt.shape) == (1, k["table_width"]) and pt.dtype == torch.int32
    assert pt[0, 0].item() == seq.page_table[0]
    assert pt[0, k["unused_index"]].item() == k["unused_value"]
    assert torch.equal(pt, ref.page_table_tensor(seq.page_table, k["table_width"]))


def test_page_table_overflow_raises_index_error_like_reference():
    seq = SequenceKVState()
    seq.page_table = [5, 6, 7]
    with pytest.raises(IndexError):
        ref.page_table_tensor(seq.page_table, 2)
    with pytest.raises(IndexError):
        seq.to_page_table_tensor(2, "cpu")


def test_last_page_slot_and_needs_new_page_over_lengths():
    for n in range(0, 70):
        s, m = SequenceKVState(), ref.SeqModel()
        s.seq_len = m.seq_len = n
        s.page_table = m.page_table = list(range((n + 15) // 16))
        assert s.last_page_slot == m.last_page_slot()
        assert s.needs_new_page() == m.needs_new_page()


def test_prefill_slot_mapping_matches_oracle():
    g = torch.Generator().manual_seed(101)
    c = cpu_cache(512)
    c.shuffle_free_list(g)
    pool = ref.PoolModel(512, list(c._free_pages))
    lens = torch.randint(1, 513, (8,), generator=g).tolist()
    seqs = [SequenceKVState() for _ in lens]
    slots = prefill_slot_mapping(c, seqs, lens)
    msq = [ref.SeqModel() for _ in lens]
    want = [x for s, n in zip(msq, lens) for x in s.add_tokens(pool, n)]
    assert slots.tolist() == want
    assert [s.page_table for s in seqs] == [m.page_table for m in msq]
    assert slots.unique().numel() == slots.numel()
    assert np.array_equal(slot_mapping_for(seqs[0], 0, lens[0]), np.array(want[:lens[0]]))


def test_kernels_refuse_cpu_tensors():
    c = cpu_cache(4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        c.write_kv(0, 1, 0, torch.zeros(1, 256), torch.zeros(1, 256))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        c.gather(0, torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))


def test_kvcache_errors_like_reference():
    kv = KVCache(8, torch.device("cpu"))
    with pytest.raises(ValueError):
        kv.append(0, torch.zeros(1, 2, 256), torch.zeros(1, 2, 256))  # a GDN layer
    with pytest.raises(AssertionError, match="KV cache overflow: 9 > 8"):
        kv.append(3, torch.zeros(9, 2, 256), torch.zeros(9, 2, 256))
    assert kv.memory_bytes == 15 * 2 * 8 * 2 * 256 * 2
    kv.advance(3)
    k, v = kv.get(59)
    assert k.shape == (3, 2, 256) and kv.current_len == 3
    kv.reset()
    assert kv.current_len == 0
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        kv.append(3, torch.zeros(1, 2, 256), torch.zeros(1, 2, 256))


def test_get_kv_by_layer_views_alias_the_pool():
    c = cpu_cache(4)
    k, v = c.get_kv_by_layer(0)
    assert k.shape == (4, 16, 1, 256) and k.data_ptr() == c.cache[0, 0].data_ptr()
    assert v.data_ptr() == c.cache[0, 1].data_ptr()


@pytest.mark.parametrize("free_bytes,dtype,want", [
    # the reference's own case (muserve/kv_cache.py:60-73): 60 layers, 1 KV
    # head of 256, 2-byte elements -> 983,040 bytes a page; 288e9 free bytes
    # leave 259.2e9 after the 10 % reserve -> 263,671.875 pages
    (288_000_000_000, torch.float16, 263_671),
    (288_000_000_000, torch.bfloat16, 263_671),
    # fp8: 256 code bytes + a 4-byte scale per (token, head) -> 499,200 bytes
    # a page; 259.2e9 / 499,200 = 519,230.77
    (288_000_000_000, torch.float8_e4m3fn, 519_230),
    # the reserve is int(free * 0.10), taken before the division:
    # 1,000,000,007 - 100,000,000 = 900,000,007 -> 915.52 -> the 1024 floor
    (1_000_000_007, torch.float16, 1024),
    # just above the floor: 1,200,000,000 - 120,000,000 = 1.08e9 -> 1098.63
    (1_200_000_000, torch.bfloat16, 1098),
])
def test_estimate_pages_closed_form(monkeypatch, free_bytes, dtype, want):
    """_estimate_pages against the reference's arithmetic worked out by hand
    (elements sized by the dtype; fp8 counts its per-token scale)."""
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (free_bytes, 2 * free_bytes))
    assert PagedKVCache._estimate_pages("cuda:0", 1, dtype) == want
