"""Pins for the paged oracle: write/gather round trip (the exact-match check of
muserve/scripts/test_kv_cache.py:58-84) and gathers vs a per-position brute force."""
import numpy as np
import torch

from oracle import paged as ref


def test_write_read_exact_round_trip():
    cache = torch.zeros(2, 2, 100, 16, 1, 256, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 256, generator=g).bfloat16()
    v = torch.randn(1, 256, generator=g).bfloat16()
    ref.write_kv(cache, 0, 42, 0, k, v)
    assert (cache[0, 0, 42, 0] - k).abs().max().item() == 0.0
    assert (cache[0, 1, 42, 0] - v).abs().max().item() == 0.0


def test_gathers_match_bruteforce():
    rng = np.random.default_rng(2)
    g = torch.Generator().manual_seed(2)
    P, B = 64, 5
    plane = torch.randn(P, 16, 2, 8, generator=g).bfloat16()
    lens = rng.integers(0, 120, B)
    width = 9
    bt = np.stack([rng.permutation(P)[:width] for _ in range(B)]).astype(np.int32)
    starts = np.minimum(rng.integers(0, 40, B), np.maximum(lens - 1, 0)).astype(np.int32)
    for out_len, st in [(144, None), (37, starts)]:
        want = ref.gather_bruteforce(plane.view(torch.int16).numpy(), bt, lens, out_len,
                                     None if st is None else st)
        got = ref.gather_padded(plane, torch.from_numpy(bt), torch.from_numpy(lens), out_len,
                                None if st is None else torch.from_numpy(st))
        assert np.array_equal(got.view(torch.int16).numpy(), want)
    packed = ref.gather_packed(plane, torch.from_numpy(bt), torch.from_numpy(lens))
    full = ref.gather_bruteforce(plane.view(torch.int16).numpy(), bt, lens, 144)
    for b in range(B):
        assert np.array_equal(packed[b].view(torch.int16).numpy(), full[b, :lens[b]])


def test_append_skips_minus_one_and_covers_layers():
    cache = torch.zeros(3, 2, 4, 16, 1, 8, dtype=torch.bfloat16)
    k = torch.arange(3 * 4 * 8, dtype=torch.float32).reshape(3, 4, 1, 8).bfloat16()
    ref.append(cache, torch.tensor([5, -1, 63, 0]), k, -k)
    for l in range(3):
        assert torch.equal(cache[l, 0].reshape(64, 1, 8)[[5, 63, 0]], k[l, [0, 2, 3]])
        assert torch.equal(cache[l, 1].reshape(64, 1, 8)[[5, 63, 0]], -k[l, [0, 2, 3]])
    assert cache[:, :, 0, 1:].abs().sum() == 0 or True
    written = {5, 63, 0}
    for s in range(64):
        if s not in written:
            assert cache[:, :, s // 16, s % 16].abs().sum() == 0
