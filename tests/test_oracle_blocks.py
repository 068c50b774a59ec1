"""Pins for the block-manager model: an independent timestamp-LRU brute force
agrees with the OrderedDict model on random traces, and the invariants
(refcount = holders, pages partitioned into free / LRU / held, table <->
cached pages) hold after every operation."""
import numpy as np
import pytest

import bench
from oracle.blocks import OK, OOM, BlockManagerModel, TimestampLRUModel
from oracle.sha import page_hashes


def trace(seed, n, P, batch):
    reqs = bench.prefix_requests(n, seed=seed, n_templates=6, template_len=64, suffix=(1, 70),
                                 zipf_s=1.1)
    hashes = [page_hashes(x) for x in reqs]
    return reqs, hashes, bench.prefix_ops(n, batch)


@pytest.mark.parametrize("seed,P,batch", [(1, 60, 3), (2, 35, 6), (3, 200, 8), (4, 30, 4)])
def test_models_agree_and_invariants_hold(seed, P, batch):
    reqs, hashes, ops = trace(seed, 80, P, batch)
    free = list(np.random.default_rng(seed).permutation(P))
    a, b = BlockManagerModel(P, free), TimestampLRUModel(P, free)
    statuses = []
    for ops_b in ops:
        for op in ops_b:
            if op >= 0:
                ra = a.admit(op, hashes[op], len(reqs[op]))
                rb = b.admit(op, hashes[op], len(reqs[op]))
                assert ra == rb, op
                statuses.append(ra["status"])
                if ra["status"] != OK:
                    continue
            else:
                r = -op - 1
                if r not in a.reqs:
                    continue
                a.release(r)
                b.release(r)
            a.check_invariants()
            assert a.free == b.free and a.ref == b.ref and a.hash == b.hash
            assert a.lru_order() == b.lru_order() and a.evicted == b.evicted
    assert OK in statuses
    if P <= 45:
        assert OOM in statuses and a.evicted


def test_hand_trace():
    """4 pages. A: 2 full pages + 1 token -> pages 3,2 (table), 1 (COW copy).
    Release A: child's copy 1 -> free, parent's partial 2... """
    m = BlockManagerModel(4)
    r = m.admit(0, [11, 22], 33)     # 33 tokens: 2 full pages, partial third
    assert r["status"] == OK and r["hits"] == 0
    assert r["table"] == [3, 2, 1] and r["cow_src"] == 1 and r["cow_dst"] == 0
    assert m.ref == [1, 1, 2, 2]     # child holds 3, 2 and its copy 0; parent 3, 2, 1
    m.release(0)                     # child tail first: 0 free; 2, 3 to 1; parent: 1 free, 2, 3 -> LRU
    assert m.free == [0, 1] and m.lru_order() == [2, 3]
    r = m.admit(1, [11, 99], 32)     # shares page 3 (hash 11), misses 99
    assert r["hits"] == 1 and r["table"] == [3, 1] and r["cow_src"] == -1
    assert m.lru_order() == [2]      # 3 pinned again, 2 still evictable
    r = m.admit(2, [55], 16)         # needs 1 page: free has [0]
    assert r["table"] == [0]
    r = m.admit(3, [77], 16)         # free empty: evicts 2 (the LRU page), hash 22 leaves
    assert r["table"] == [2] and m.evicted == [2] and 22 not in m.table
    assert m.admit(4, [88], 16)["status"] == OOM
    m.check_invariants()
