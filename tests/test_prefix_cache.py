"""PrefixCache (host) vs the OrderedDict model of muserve/model/prefix_cache.py."""
import numpy as np
import torch

from muserve_amd.model.prefix_cache import PrefixCache
from oracle.lru import PrefixCacheModel
from oracle.sha import hash_tokens


def _ids(rng, n):
    return torch.from_numpy(rng.integers(0, 151936, n, dtype=np.int64))


def test_key_is_reference_formula():
    ids = torch.arange(40, dtype=torch.int64)
    assert PrefixCache._hash_tokens(ids) == hash_tokens(ids.numpy())
    assert PrefixCache._prefix_keys(ids.numpy().tobytes(), 8, [5, 40, 17]) == {
        n: hash_tokens(ids.numpy()[:n]) for n in (5, 17, 40)}


def test_hand_trace_eviction_order():
    # capacity 2: store A, B; lookup A (A -> MRU); store C evicts B (the LRU)
    base = torch.arange(100, dtype=torch.int64)
    pc = PrefixCache(max_entries=2)
    hidden = torch.zeros(3)
    pc.store(base, 10, hidden, [None])
    pc.store(base + 1, 20, hidden, [None])
    hit = pc.lookup(base, torch.device("cpu"))
    assert hit is not None and hit[0] == 10
    pc.store(base + 2, 30, hidden, [None])
    assert list(pc._cache) == [hash_tokens((base + 0).numpy()[:10]),
                               hash_tokens((base + 2).numpy()[:30])]
    assert pc.lookup(base + 1, torch.device("cpu")) is None  # B was evicted
    assert len(pc) == 2


def test_random_traces_match_model():
    rng = np.random.default_rng(3)
    templates = [_ids(rng, 64) for _ in range(6)]
    pc, model = PrefixCache(max_entries=5), PrefixCacheModel(5)
    for step in range(400):
        t = templates[int(rng.integers(0, 6))]
        ids = torch.cat([t[:int(rng.integers(8, 64))], _ids(rng, int(rng.integers(0, 8)))])
        if rng.random() < 0.5:
            plen = int(rng.integers(1, len(ids) + 1))
            pc.store(ids, plen, torch.zeros(1), [torch.ones(2), None])
            model.store(ids.numpy(), plen)
        else:
            hit = pc.lookup(ids, torch.device("cpu"))
            want = model.lookup(ids.numpy())
            assert (hit[0] if hit else None) == want
        assert list(pc._cache) == model.keys()
        assert [e["prefix_len"] for e in pc._cache.values()] == list(model.entries.values())


def test_store_existing_key_only_touches():
    pc = PrefixCache(max_entries=4)
    ids = torch.arange(30, dtype=torch.int64)
    pc.store(ids, 10, torch.zeros(1), [None])
    pc.store(ids + 5, 10, torch.zeros(1), [None])
    pc.store(ids, 10, torch.ones(1), [None])
    assert list(pc._cache)[-1] == hash_tokens(ids.numpy()[:10])
    assert pc._cache[hash_tokens(ids.numpy()[:10])]["hidden"].item() == 0.0  # value not replaced
    assert pc.memory_mb() == 2 * 4 / 1024 / 1024
    pc.clear()
    assert len(pc) == 0
