"""GPU per-page SHA-256 prefix hashes vs hashlib."""
import numpy as np
import pytest
import torch

from muserve_amd.prefix_hash import as_u64, page_hashes
from oracle import sha as ref
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [np.int64, np.int32])
def test_page_hashes_match_hashlib(dtype):
    rng = np.random.default_rng(104)
    lens = [0, 5, 16, 17, 31, 32, 300, 1000] + rng.integers(0, 700, 300).tolist()
    case(f"page hashes {len(lens)} requests {np.dtype(dtype).name}")
    ids = [rng.integers(0, 151936, n).astype(dtype) for n in lens]
    flat = np.concatenate(ids)
    cu = np.concatenate([[0], np.cumsum(lens)])
    h, cu_p = page_hashes(torch.from_numpy(flat).to(DEV), cu)
    got = as_u64(h)
    for r, x in enumerate(ids):
        want = ref.page_hashes(x)
        assert got[cu_p[r]:cu_p[r + 1]].tolist() == want, r


def test_page_hashes_workgroup_without_pages():
    # 32 requests of the first workgroup have no full page (it runs no step);
    # the second mixes empty, partial and long requests
    lens = [3] * 32 + [40, 0, 15, 600, 16, 2047]
    case(f"page hashes {len(lens)} requests, a workgroup without pages")
    rng = np.random.default_rng(5)
    ids = [rng.integers(0, 151936, n).astype(np.int64) for n in lens]
    cu = np.concatenate([[0], np.cumsum(lens)])
    h, cu_p = page_hashes(torch.from_numpy(np.concatenate(ids)).to(DEV), cu)
    got = as_u64(h)
    assert cu_p[32] == 0
    for r, x in enumerate(ids):
        assert got[cu_p[r]:cu_p[r + 1]].tolist() == ref.page_hashes(x), r
