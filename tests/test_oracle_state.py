"""The state-pool and host-tier oracle (oracle/state.py) against per-element
pure-Python brute force on small pools: slot gather / scatter, and the
layered block pack / unpack (zeros for, or skipping of, ids outside the pool)."""
import numpy as np
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


def _bf16_ulp(v):
    mag = np.maximum(np.abs(v), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(mag)) - 7)


def test_conv_decode_matches_the_reference_formula():
    # width 3 is the reference's [C, K-1] state: its fp32 F.conv1d + SiLU
    # (qwen35_layer_v2.py:175-199) vs the float64 oracle, one request
    g = torch.Generator().manual_seed(3)
    C = 64
    for _ in range(20):
        st = torch.randn(C, 3, generator=g).bfloat16()
        x = torch.randn(1, C, generator=g).bfloat16()
        w = (0.5 * torch.randn(C, 1, 4, generator=g)).bfloat16()
        ref_out, ref_state = state.conv_decode_reference_fp32(st, x, w)
        pool = st.unsqueeze(0).clone()
        want = state.conv_decode(pool, torch.tensor([0]), x, w)
        assert torch.equal(pool[0], ref_state)                       # the shift is exact
        err = (ref_out.double() - want).abs().numpy()
        assert (err <= _bf16_ulp(want.numpy())).all()                 # one bf16 rounding apart


def test_conv_decode_closed_forms_and_width_4():
    g = torch.Generator().manual_seed(4)
    C, S = 16, 5
    pool = torch.randn(S, C, 4, generator=g).bfloat16()
    x = torch.randn(2, C, generator=g).bfloat16()
    slots = torch.tensor([3, 1])
    for k in range(4):  # one-hot weights pick one input: silu of it, exactly
        w = torch.zeros(C, 4)
        w[:, k] = 1.0
        p = pool.clone()
        out = state.conv_decode(p, slots, x, w.bfloat16())
        for b, s in enumerate(slots.tolist()):
            pick = pool[s, :, 1 + k].double() if k < 3 else x[b].double()  # width 4: last 3 columns
            assert torch.equal(out[b], pick * torch.sigmoid(pick))
            assert torch.equal(p[s], torch.cat([pool[s, :, 1:], x[b].unsqueeze(1)], 1))
        untouched = [i for i in range(S) if i not in (3, 1)]
        assert torch.equal(p[untouched], pool[untouched])
    out = state.conv_decode(pool.clone(), slots, x, torch.zeros(C, 4).bfloat16())
    assert torch.count_nonzero(out) == 0
    # requests are independent: each equals the one-request computation on its slot
    w = torch.randn(C, 4, generator=g).bfloat16()
    p = pool.clone()
    both = state.conv_decode(p, slots, x, w)
    for b, s in enumerate(slots.tolist()):
        q = pool.clone()
        assert torch.equal(state.conv_decode(q, torch.tensor([s]), x[b:b + 1], w)[0], both[b])
    # a slot outside the pool: zeros, pool unchanged
    q = pool.clone()
    assert torch.count_nonzero(state.conv_decode(q, torch.tensor([9]), x[:1], w)) == 0
    assert torch.equal(q, pool)
