"""Host-tier bookkeeping on the CPU: the pinned arena's range allocator
(muserve_amd/memory/host_tier.py), exercised on a pageable buffer, against a
byte-map brute force."""
import numpy as np
import pytest

from muserve_amd.memory.host_tier import ALIGN, PinnedArena


def test_first_fit_and_coalescing():
    a = PinnedArena(16 * ALIGN, pinned=False)
    x = a.alloc(1)            # rounds up to one unit
    y = a.alloc(3 * ALIGN)
    z = a.alloc(2 * ALIGN + 5)
    assert (x, y, z) == (0, ALIGN, 4 * ALIGN)
    assert a.free_bytes() == 9 * ALIGN
    a.free(y, 3 * ALIGN)
    assert a.alloc(2 * ALIGN) == ALIGN          # first fit reuses the hole
    a.free(ALIGN, 2 * ALIGN)
    a.free(x, 1)
    a.free(z, 2 * ALIGN + 5)
    assert a._free == [(0, 16 * ALIGN)]         # everything merged back
    assert a.alloc(17 * ALIGN) is None
    with pytest.raises(ValueError):
        a.free(0, ALIGN)                        # double free


def test_random_alloc_free_against_byte_map():
    rng = np.random.default_rng(7)
    units = 64
    a = PinnedArena(units * ALIGN, pinned=False)
    used = np.zeros(units, dtype=bool)
    live = []
    for _ in range(3000):
        if live and rng.random() < 0.45:
            off, n = live.pop(int(rng.integers(0, len(live))))
            a.free(off, n)
            used[off // ALIGN: off // ALIGN + -(-n // ALIGN)] = False
        else:
            n = int(rng.integers(1, 6 * ALIGN))
            k = -(-n // ALIGN)
            off = a.alloc(n)
            # brute force: the first run of k free units
            runs = [i for i in range(units - k + 1) if not used[i:i + k].any()]
            if off is None:
                assert not runs
                continue
            assert off == runs[0] * ALIGN
            used[runs[0]:runs[0] + k] = True
            live.append((off, n))
        assert a.free_bytes() == (~used).sum() * ALIGN
        assert all(a._free[i][0] + a._free[i][1] < a._free[i + 1][0]
                   for i in range(len(a._free) - 1))  # sorted, never adjacent
