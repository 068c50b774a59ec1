"""Pins for prefix hashing: hashlib vs FIPS 180 vectors; the page-hash chain vs
hashing each prefix from scratch; the kernels' SHA-256 (mkv_common.h, host
build) vs hashlib."""
import hashlib
import json

import numpy as np
import pytest

from oracle import sha as ref
from tests.helpers import GOLDEN, hostcheck, np_ptr

FIPS = json.loads((GOLDEN / "sha256_fips.json").read_text())


@pytest.mark.parametrize("vec", FIPS, ids=lambda v: v["msg_ascii"][:8] or "empty")
def test_hashlib_matches_fips_vectors(vec):
    msg = vec["msg_ascii"].encode() * vec.get("repeat", 1)
    assert hashlib.sha256(msg).hexdigest() == vec["sha256"]


def host_page_hashes(ids: np.ndarray) -> list[int]:
    ids = np.ascontiguousarray(ids)
    out = np.zeros(len(ids) // 16, np.uint64)
    hostcheck().hc_page_hashes(np_ptr(ids), len(ids), ids.itemsize, np_ptr(out))
    return [int(v) for v in out]


@pytest.mark.parametrize("dtype", [np.int64, np.int32])
def test_page_chain_equals_prefix_hashes(dtype):
    rng = np.random.default_rng(1)
    for n in [0, 15, 16, 17, 64, 100, 333]:
        ids = rng.integers(0, 151936, n).astype(dtype)
        want = ref.page_hashes_from_scratch(ids)
        assert ref.page_hashes(ids) == want
        assert host_page_hashes(ids) == want


def test_page_hash_is_prefix_cache_key():
    ids = np.arange(48, dtype=np.int64)
    h = ref.page_hashes(ids)
    key = hashlib.sha256(ids[:32].tobytes()).hexdigest()[:16]  # prefix_cache.py:31-34
    assert h[1] == int(key, 16) and format(h[1], "016x") == key
