"""Guards against caller mistakes that the kernels catch on the device:
packed-gather offsets that leave too little room, and repeated slots under
the opt-in duplicate check. Each is reported as MkvDeviceError at the next
check, and nothing outside the caller's buffers is written."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kv_cache import PagedKVCache, SequenceKVState, prefill_slot_mapping
from muserve_amd.state_pool import StatePool
from tests.gpu_util import DEV, bits16, case

pytestmark = pytest.mark.gpu


def _filled_pool(dtype, lens, seed):
    g = torch.Generator().manual_seed(seed)
    cache = PagedKVCache(64, num_layers=2, dtype=dtype, device=DEV, verbose=False)
    seqs = [SequenceKVState() for _ in lens]
    slots = prefill_slot_mapping(cache, seqs, lens)
    T = sum(lens)
    k = torch.randn(2, T, 1, 256, generator=g).bfloat16()
    v = torch.randn(2, T, 1, 256, generator=g).bfloat16()
    cache.append(slots, k.to(DEV), v.to(DEV))
    W = max(len(s.page_table) for s in seqs)
    bt = torch.zeros(len(seqs), W, dtype=torch.int32)
    for b, s in enumerate(seqs):
        bt[b, :len(s.page_table)] = torch.tensor(s.page_table, dtype=torch.int32)
    cache.check_errors()
    return cache, bt.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_packed_gather_keeps_inside_offsets_and_buffer(dtype):
    lens = [40, 25, 33]
    case(f"packed gather with overlapping offsets and a short buffer, {dtype}")
    cache, bt, sl = _filled_pool(dtype, lens, 7)
    # reference: consistent offsets
    cu = torch.tensor([0, 40, 65, 98], dtype=torch.int64, device=DEV)
    want_k, want_v = cache.gather(0, bt, sl, out_len=40, cu_out=cu)
    cache.check_errors()
    # sequence 0 (40 rows) is given 30 (offsets 0, 30, ...), and sequence 2
    # (33 rows from row 55) runs past the buffer's 80 rows: both are cut and
    # flagged, and the rows past the buffer keep their canary
    cu_bad = torch.tensor([0, 30, 55, 88], dtype=torch.int64, device=DEV)
    canary = 0x1234
    k_out = torch.zeros(96, 1, 256, dtype=torch.int16, device=DEV)
    v_out = torch.zeros(96, 1, 256, dtype=torch.int16, device=DEV)
    k_out[80:] = canary
    v_out[80:] = canary
    k_view = k_out.view(torch.bfloat16)[:80]
    v_view = v_out.view(torch.bfloat16)[:80]
    cache.gather(0, bt, sl, out_len=40, cu_out=cu_bad, out=(k_view, v_view))
    with pytest.raises(_lib.MkvDeviceError, match="inconsistent offsets"):
        cache.check_errors()
    assert (k_out[80:] == canary).all() and (v_out[80:] == canary).all()
    # the rows that fit hold the right data
    for got, want in ((bits16(k_view), bits16(want_k)), (bits16(v_view), bits16(want_v))):
        assert torch.equal(got[0:30], want[0:30])    # sequence 0, cut to 30 rows
        assert torch.equal(got[30:55], want[40:65])  # sequence 1, whole
        assert torch.equal(got[55:80], want[65:90])  # sequence 2, cut by the buffer
    # a negative offset writes nothing for that sequence
    cu_neg = torch.tensor([-5, 40, 65, 98], dtype=torch.int64, device=DEV)
    fresh_k, fresh_v = cache.gather(0, bt, sl, out_len=40, cu_out=cu_neg)
    with pytest.raises(_lib.MkvDeviceError):
        cache.check_errors()
    assert torch.equal(bits16(fresh_k)[40:], bits16(want_k)[40:])


def test_packed_gather_exact_room_is_not_flagged():
    lens = [16, 1, 31]
    case("packed gather whose offsets leave exactly the rows needed")
    cache, bt, sl = _filled_pool(torch.bfloat16, lens, 8)
    cu = torch.tensor([0, 16, 17, 48], dtype=torch.int64, device=DEV)
    k, v = cache.gather(0, bt, sl, out_len=31, cu_out=cu)
    cache.check_errors()
    kk, _ = cache.gather(0, bt, sl, out_len=32)
    assert torch.equal(bits16(k)[17:48], bits16(kk)[2, :31])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_duplicate_slot_in_append_is_reported_when_checked(dtype):
    case(f"append with a repeated slot, duplicate check on and off, {dtype}")
    cache = PagedKVCache(16, num_layers=1, dtype=dtype, device=DEV, verbose=False)
    k = torch.randn(4, 1, 256, device=DEV).bfloat16()
    slots = torch.tensor([3, 17, -1, 3], dtype=torch.int64, device=DEV)
    cache.check_unique = False  # the default: not checked
    cache.append(slots, k, k, layer=0)
    cache.check_errors()
    cache.check_unique = True
    cache.append(slots, k, k, layer=0)
    with pytest.raises(_lib.MkvDeviceError, match="appears more than once"):
        cache.check_errors()
    # unique slots (and repeated -1 skips) pass; the bitmap was left clear
    for _ in range(2):
        cache.append(torch.tensor([3, -1, 17, -1], dtype=torch.int64, device=DEV), k, k, layer=0)
        cache.check_errors()


def test_duplicate_slot_in_state_scatter_is_reported_when_checked():
    case("state pool scatter / reset with a repeated slot under the duplicate check")
    pool = StatePool(num_layers=2, num_slots=8, state_shape=(4, 64), conv_shape=(16, 4),
                     device=DEV)
    pool.check_unique = True
    st = torch.randn(3, 4, 64, device=DEV)
    cv = torch.randn(3, 16, 4, device=DEV).bfloat16()
    pool.scatter(1, torch.tensor([2, 5, 7], dtype=torch.int32), st, cv)
    pool.check_errors()
    pool.scatter(1, torch.tensor([2, 5, 2], dtype=torch.int32), st, cv)
    with pytest.raises(_lib.MkvDeviceError, match="appears more than once"):
        pool.check_errors()
    pool.reset([4, 4])
    with pytest.raises(_lib.MkvDeviceError, match="appears more than once"):
        pool.check_errors()
    pool.reset([4, 6])
    pool.check_errors()


def test_check_unique_entry_point_directly():
    case("mkv_check_unique on int32 and int64 lists, limits and skips")
    err = _lib.DeviceErrors(DEV)
    chk = _lib.UniqueCheck(DEV, 1000)
    rng = np.random.default_rng(3)
    ids = torch.from_numpy(rng.permutation(1000)[:700].astype(np.int64)).to(DEV)
    chk.run(ids, err)
    chk.run(ids.to(torch.int32), err)
    err.check()
    # out-of-range ids are ignored, even repeated
    chk.run(torch.tensor([1000, 1000, -7, -7, 5], dtype=torch.int64, device=DEV), err)
    err.check()
    dup = torch.cat([ids, ids[123:124]])
    chk.run(dup, err)
    with pytest.raises(_lib.MkvDeviceError):
        err.check()
    assert int(chk.bits.count_nonzero()) == 0


def test_stream_of_is_torchs_current_stream():
    # every entry point is launched on the stream stream_of returns: torch's
    # current stream of the device, also inside a stream context
    case("stream_of against torch.cuda.current_stream")
    assert _lib.stream_of(DEV) == torch.cuda.current_stream(DEV).cuda_stream
    side = torch.cuda.Stream(DEV)
    with torch.cuda.stream(side):
        assert _lib.stream_of(DEV) == side.cuda_stream
        assert _lib.stream_of(torch.device("cuda")) == side.cuda_stream
    assert _lib.stream_of(DEV) == torch.cuda.current_stream(DEV).cuda_stream
