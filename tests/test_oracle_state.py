"""The state-pool and host-tier oracle (oracle/state.py) against per-element
pure-Python brute force on small pools: slot gather / scatter, and the
layered block pack / unpack (zeros for, or skipping of, ids outside the pool)."""
import torch

from oracle import state


def _pool(planes, blocks, width, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-1000, 1000, (planes, blocks, width), generator=g)


def test_gather_scatter_brute_force():
    pool = _pool(3, 9, 5, 1)
    slots = torch.tensor([4, 0, 8, 4])
    for layer in range(3):
        got = state.gather(pool, layer, slots)
        for i, s in enumerate(slots.tolist()):
            assert got[i].tolist() == pool[layer, s].tolist()
    x = torch.arange(3 * 5).view(3, 5)
    uniq = torch.tensor([7, 2, 5])
    p2 = pool.clone()
    state.scatter(p2, 1, uniq, x)
    for s in range(9):
        for layer in range(3):
            want = x[uniq.tolist().index(s)] if layer == 1 and s in uniq.tolist() else pool[layer, s]
            assert p2[layer, s].tolist() == want.tolist()


def test_pack_unpack_brute_force():
    pool = _pool(4, 11, 6, 2)
    ids = torch.tensor([10, 3, -1, 0, 11, 7])
    packed = state.pack_blocks(pool, ids)
    assert packed.shape == (4, 6, 6)
    for z in range(4):
        for i, b in enumerate(ids.tolist()):
            want = pool[z, b].tolist() if 0 <= b < 11 else [0] * 6
            assert packed[z, i].tolist() == want
    back = torch.full_like(pool, 5)
    state.unpack_blocks(back, ids, packed)
    for z in range(4):
        for b in range(11):
            want = pool[z, b].tolist() if b in (10, 3, 0, 7) else [5] * 6
            assert back[z, b].tolist() == want
    # a round trip through different blocks moves exactly those blocks
    other = torch.tensor([1, 2, 9, 4, 5, 6])
    moved = torch.zeros_like(pool)
    state.unpack_blocks(moved, other, state.pack_blocks(pool, torch.tensor([10, 3, 8, 0, 1, 7])))
    assert moved[:, [1, 2, 9, 4, 5, 6]].tolist() == pool[:, [10, 3, 8, 0, 1, 7]].tolist()
