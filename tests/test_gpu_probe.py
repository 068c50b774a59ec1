"""The access-pattern probes (mkv_probe_*) that bench.py --workload ceilings
times: the two writing probes write exactly what their header says (checked
against torch on the same bytes), page ids outside the pool are skipped, and
the read-only probes leave their sink untouched (the loads are kept alive by
a store that no realistic data triggers)."""
import pytest
import torch

from muserve_amd import _lib
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


def _stream():
    return _lib.stream_of(DEV)


def test_fill_writes_zeros_and_nothing_else():
    case("mkv_probe_fill: 3 tiles inside a guarded buffer")
    buf = torch.full((4096 * 5,), 0xA5, dtype=torch.uint8, device=DEV)
    _lib.call("mkv_probe_fill", buf[4096:].data_ptr(), 3 * 4096, _stream())
    torch.cuda.synchronize()
    got = buf.cpu()
    assert (got[4096:4 * 4096] == 0).all()
    assert (got[:4096] == 0xA5).all() and (got[4 * 4096:] == 0xA5).all()


def test_scatter_pages_against_torch():
    g = torch.Generator().manual_seed(5)
    planes, npages, dpages = 3, 6, 10
    case(f"mkv_probe_scatter_pages: {planes} planes, {npages} pages into {dpages}, two skipped")
    src = torch.randint(0, 256, (planes, npages * 8192), dtype=torch.uint8, generator=g)
    pages = torch.tensor([7, 2, -1, 9, 10, 0], dtype=torch.int32)  # -1 and 10 lie outside
    dst0 = torch.randint(0, 256, (planes, dpages * 4096), dtype=torch.uint8, generator=g)
    dst = dst0.to(DEV)
    src_d, pages_d = src.to(DEV), pages.to(DEV)  # held until the launch has run
    _lib.call("mkv_probe_scatter_pages", src_d.data_ptr(), src.stride(0), dst.data_ptr(),
              dst.stride(0), dpages, pages_d.data_ptr(), npages, planes, _stream())
    torch.cuda.synchronize()
    want = dst0.clone()
    for y in range(planes):
        for x, p in enumerate(pages.tolist()):
            if 0 <= p < dpages:
                pair = src[y, x * 8192:(x + 1) * 8192].view(256, 2, 16)
                want[y, p * 4096:(p + 1) * 4096] = (pair[:, 0] ^ pair[:, 1]).reshape(-1)
    assert torch.equal(dst.cpu(), want)


@pytest.mark.parametrize("page_bytes", [8192, 4096])
@pytest.mark.parametrize("walk,nt", [(0, 1), (1, 0), (1, 1)])
def test_read_probes_write_nothing(page_bytes, walk, nt):
    n_pool, n = 40, 300
    case(f"mkv_probe_read_pages: {page_bytes} B pages, walk {walk}, nt {nt}")
    g = torch.Generator().manual_seed(page_bytes + walk)
    kp = torch.randint(0, 256, (n_pool * page_bytes,), dtype=torch.uint8, generator=g).to(DEV)
    vp = torch.randint(0, 256, (n_pool * page_bytes,), dtype=torch.uint8, generator=g).to(DEV)
    pages = torch.randint(-3, n_pool + 3, (n,), dtype=torch.int32, generator=g).to(DEV)
    sink = torch.zeros(16384, dtype=torch.uint8, device=DEV)
    _lib.call("mkv_probe_read_pages", kp.data_ptr(), vp.data_ptr(), page_bytes, n_pool,
              pages.data_ptr(), n, walk, nt, sink.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert int(sink.count_nonzero()) == 0
