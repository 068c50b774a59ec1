"""mkv_decode_attention_bf16_noalloc (the library's static scratch, nothing
allocated) against mkv_decode_attention_bf16 (the caller's workspace), both
called through the C ABI: two calls in a row, the second with a smaller
input, each output equal bit for bit (the same kernels over the same work
split). The rejection of an unsupported shape is a host-side check, tested
without a GPU in tests/test_abi.py."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kernels import attention as A
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


def _inputs(seed, lens, Hq=4, Hkv=1):
    """Pool pages in a seeded random order, K/V/q ~N(0,1) bf16 on the device."""
    rng = np.random.default_rng(seed)
    pages = [-(-int(n) // 16) for n in lens]
    P = sum(pages) + 3
    perm = rng.permutation(P)
    table = np.zeros((len(lens), max(1, max(pages))), dtype=np.int32)
    at = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[at:at + n]
        at += n
    gen = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn(P, 16, Hkv, 256, generator=gen, device=DEV).bfloat16()
    v = torch.randn(P, 16, Hkv, 256, generator=gen, device=DEV).bfloat16()
    q = torch.randn(len(lens), 1, Hq, 256, generator=gen, device=DEV).bfloat16()
    return (q, k, v, torch.from_numpy(np.asarray(lens, dtype=np.int32)).to(DEV),
            torch.from_numpy(table).to(DEV))


def _call(fn, q, k, v, lens, table, max_len, out, ws=None):
    shared = [] if ws is None else [0]  # the workspace entry point's shared_pages bound
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), k.shape[0], *shared, k.shape[2],
            q.shape[2], 256,
            table.data_ptr(), table.stride(0), table.shape[1], lens.data_ptr(), q.shape[0],
            max_len, 256 ** -0.5, out.data_ptr()]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    _lib.call(fn, *args, A._errword(DEV).ptr(), _lib.stream_of(DEV))


def test_noalloc_equals_the_workspace_entry_point_on_two_calls():
    rng = np.random.default_rng(102)
    # the decode configuration's lengths (lognormal, median 4096, clipped to
    # 32768: most sequences cut between waves, the merge kernel used), then a
    # smaller batch of shorter sequences (empty ones included) on the same
    # scratch, which keeps the first call's contents
    big = np.clip(np.round(rng.lognormal(np.log(4096.0), 1.0, 256)), 1, 32768).astype(np.int64)
    small = rng.integers(0, 3000, 40)
    small[:2] = (0, 1)
    for seed, lens in ((71, big), (72, small)):
        case(f"decode attention no-alloc vs workspace: batch {len(lens)}, "
             f"{int(lens.sum())} tokens, max {int(lens.max())}")
        q, k, v, ld, table = _inputs(seed, lens)
        max_len = int(lens.max())
        ws = torch.zeros(A.workspace_bytes(len(lens), 1, 4, max_len), dtype=torch.uint8,
                         device=DEV)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        _call("mkv_decode_attention_bf16", q, k, v, ld, table, max_len, want, ws)
        _call("mkv_decode_attention_bf16_noalloc", q, k, v, ld, table, max_len, got)
        torch.cuda.synchronize()
        A.check_errors(DEV)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        assert torch.isfinite(got.float()).all()

