"""GPU parity of the scheduler's step plan (mkv_step_plan) vs the CPU
scheduler oracle: slot mapping, positions, cu_seqlens, per-entry block tables,
lengths and rows, bit-exact, step by step over continuous-batching traces;
then the plan driving real appends, gathers and decode attention."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kernels.attention import attn_decode, check_errors as attn_errors
from muserve_amd.kv_cache import PagedKVCache
from muserve_amd.scheduler import ContinuousBatchScheduler, InferenceRequest
from oracle import attention as oatt
from oracle import paged as pg
from oracle import sched as S
from tests.gpu_util import DEV, case
from tests.test_gpu_attention import within_one_ulp

pytestmark = pytest.mark.gpu


def req(rid, n, gen):
    return InferenceRequest(request_id=rid, input_ids=list(range(n)), max_new_tokens=gen)


def check_plan(s, plan, want, step):
    n = len(want["rids"])
    if plan is None:
        assert n == 0, f"step {step}: the oracle scheduled {n} entries"
        return
    assert [r.request_id for r in plan.entries] == want["rids"], f"step {step}"
    assert plan.slot_mapping.cpu().tolist() == want["slots"], f"step {step}: slots"
    assert plan.positions.cpu().tolist() == want["positions"], f"step {step}: positions"
    assert plan.cu_seqlens.cpu().tolist() == want["cu_seqlens"], f"step {step}: cu_seqlens"
    assert plan.seq_lens.cpu().tolist() == want["lens"], f"step {step}: lens"
    assert plan.rows.cpu().tolist() == want["rows"], f"step {step}: rows"
    w = plan.block_tables.shape[1]
    tab = np.asarray(want["tables"], dtype=np.int64)
    assert np.array_equal(plan.block_tables.cpu().numpy(), tab[:, :w]), f"step {step}: tables"
    assert not tab[:, w:].any(), f"step {step}: table wider than the plan's"


@pytest.mark.parametrize("seed,pages,chunk,batch,max_seq", [
    (0, 40, 48, 6, 256), (1, 300, 4096, 16, 1024), (2, 2048, 512, 64, 4096),
    (3, 24, 33, 8, 256)])
def test_step_plan_matches_oracle(seed, pages, chunk, batch, max_seq):
    case(f"mkv_step_plan trace seed {seed}: pages {pages} chunk {chunk} batch {batch}")
    rng = np.random.default_rng(seed)
    free = rng.permutation(pages).tolist()
    pool = pg.PoolModel(pages, free)
    m = S.ChunkedSchedulerModel(batch, chunk, pool, max_seq, eos=3)
    cache = PagedKVCache(pages, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    cache._free_pages = list(free)
    s = ContinuousBatchScheduler(max_batch_size=batch, max_seq_len=max_seq, kv_cache=cache,
                                 chunked_prefill_size=chunk, eos_token_id=3)
    pending = [(i, int(rng.integers(1, max_seq // 2)), int(rng.integers(1, 60)))
               for i in range(4 * batch)]
    steps = 0
    for step in range(4000):
        while pending and rng.random() < 0.3:
            i, n, g = pending.pop(0)
            m.add(S.Req(i, n, g))
            s.add_request(req(i, n, g))
        try:
            want = m.step()
        except RuntimeError:
            with pytest.raises(RuntimeError, match="KV cache OOM"):
                s.plan_step()
            break
        plan = s.plan_step()
        check_plan(s, plan, want, step)
        toks = rng.integers(0, 64, len(want["rids"])).tolist()
        m.complete(toks)
        if plan is not None:
            s.complete_step(plan, toks)
            steps += 1
        if not pending and s.is_idle:
            break
    s.check_errors()
    assert steps > 10


def test_plan_drives_append_gather_and_decode_attention():
    """A continuous-batching trace whose every step appends its tokens' K/V
    through plan.slot_mapping; each step's decode half then runs attn_decode
    on plan.block_tables / plan.seq_lens, and every request, when it finishes,
    reads back through its last table exactly the rows appended for it."""
    case("scheduler plan -> append -> decode attention -> gather round trip")
    rng = np.random.default_rng(11)
    g = torch.Generator(device=DEV).manual_seed(11)
    pages, batch = 512, 8
    cache = PagedKVCache(pages, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    cache._free_pages = rng.permutation(pages).tolist()
    s = ContinuousBatchScheduler(max_batch_size=batch, max_seq_len=1024, kv_cache=cache,
                                 chunked_prefill_size=160)
    reqs = [req(i, int(rng.integers(1, 400)), int(rng.integers(1, 24))) for i in range(20)]
    for r in reqs:
        s.add_request(r)
    rows_k = {r.request_id: [] for r in reqs}
    checked = set()
    attn_checked = 0
    while True:
        plan = s.plan_step()
        if plan is None:    # the last requests finished and were retired
            break
        T = plan.num_tokens
        k = torch.randn(T, 1, 256, device=DEV, generator=g).bfloat16()
        v = torch.randn(T, 1, 256, device=DEV, generator=g).bfloat16()
        cache.append(plan.slot_mapping, k, v, layer=0)
        cu = plan.cu_seqlens.cpu().tolist()
        for i, r in enumerate(plan.entries):
            rows_k[r.request_id].append(k[cu[i]:cu[i + 1]].cpu())
        nd = plan.num_decode
        if nd and attn_checked < 6:
            q = torch.randn(nd, 1, 4, 256, device=DEV, generator=g).bfloat16()
            kc, vc = cache.get_kv_by_layer(0)
            out = attn_decode(q, kc, vc, plan.seq_lens[:nd], plan.block_tables[:nd])
            want = oatt.decode_attention(q[:, 0].float().cpu().numpy(),
                                         kc.float().cpu().numpy(), vc.float().cpu().numpy(),
                                         plan.seq_lens[:nd].cpu().numpy(),
                                         plan.block_tables[:nd].cpu().numpy(), 256 ** -0.5,
                                         stats=True)
            within_one_ulp(out[:, 0], want)
            attn_checked += 1
        tables = plan.block_tables.cpu()
        lens = plan.seq_lens.cpu()
        # a finished request's pages are recycled at the next plan: read it back now
        for r in s.complete_step(plan):
            i = plan.entries.index(r)
            n = int(lens[i])
            got = pg.gather_packed(cache.cache[0, 0].cpu(), tables[i:i + 1], lens[i:i + 1])[0]
            want = torch.cat(rows_k[r.request_id])
            assert got.shape[0] == n == want.shape[0] == len(r.input_ids) + len(
                r.generated_tokens) - 1
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
                f"request {r.request_id}"
            checked.add(r.request_id)
    assert s.is_idle and checked == {r.request_id for r in reqs}
    s.check_errors()
    attn_errors(DEV)
    assert attn_checked > 0


def test_malformed_entries_raise_without_faulting():
    """Entries checked on the device: pages that do not cover the tokens,
    a row outside the tables and a page id outside the pool set error bits and
    slot -1 (page -1 in the step table); offsets that do not tile leave the
    entry's tokens unwritten."""
    case("mkv_step_plan malformed entries (host-forced, all accesses in bounds)")
    i32 = dict(dtype=torch.int32, device=DEV)
    tables = torch.zeros(4, 8, **i32)
    # row, start, count, held, new, page_off, tok_off, 0
    ent = torch.tensor([[0, 0, 20, 0, 1, 0, 0, 0],      # 1 page for 20 tokens: TABLE
                        [9, 0, 4, 0, 1, 1, 20, 0],      # row 9 of 4: TABLE
                        [2, 0, 4, 0, 1, 2, 24, 0]],     # page 500 of 64: PAGE
                       **i32)
    new_pages = torch.tensor([5, 6, 500], **i32)
    T = 28
    slots = torch.full((T,), 7, dtype=torch.int64, device=DEV)
    pos = torch.full((T,), 7, dtype=torch.int64, device=DEV)
    step_tables = torch.full((3, 8), 9, **i32)
    lens = torch.full((3,), 9, **i32)
    rows = torch.full((3,), 9, **i32)
    cu = torch.full((4,), 9, dtype=torch.int64, device=DEV)
    err = torch.zeros(1, **i32)
    _lib.call("mkv_step_plan", tables.data_ptr(), 8, 8, 4, ent.data_ptr(), 3,
              new_pages.data_ptr(), 3, 64, slots.data_ptr(), pos.data_ptr(), T,
              step_tables.data_ptr(), 8, 8, lens.data_ptr(), rows.data_ptr(), cu.data_ptr(),
              err.data_ptr(), _lib.stream_of(DEV))
    torch.cuda.synchronize()
    assert err.item() == _lib.DEVERR_TABLE | _lib.DEVERR_PAGE
    assert slots.cpu().tolist() == [-1] * T
    assert pos.cpu().tolist() == list(range(20)) + list(range(4)) + list(range(4))
    assert lens.cpu().tolist() == [0, 0, 4] and rows.cpu().tolist() == [-1, -1, 2]
    assert step_tables.cpu().tolist() == [[0] * 8, [0] * 8, [-1] + [0] * 7]
    assert cu.cpu().tolist() == [0, 20, 24, 28]
    assert tables[2, 0].item() == -1     # an out-of-pool page is not recorded
    # offsets that skip tokens: the entry stays unwritten, the error is raised
    err.zero_()
    bad = torch.tensor([[0, 0, 4, 0, 1, 0, 0, 0], [1, 0, 4, 0, 1, 1, 6, 0]], **i32)
    slots.fill_(7)
    _lib.call("mkv_step_plan", tables.data_ptr(), 8, 8, 4, bad.data_ptr(), 2,
              new_pages.data_ptr(), 2, 64, slots.data_ptr(), pos.data_ptr(), 10,
              step_tables.data_ptr(), 8, 8, lens.data_ptr(), rows.data_ptr(), cu.data_ptr(),
              err.data_ptr(), _lib.stream_of(DEV))
    torch.cuda.synchronize()
    assert err.item() == _lib.DEVERR_TABLE
    assert slots[:10].cpu().tolist() == [7] * 6 + [96, 97, 98, 99]


def test_admitted_requests_get_zeroed_state_slots():
    """With a state pool attached, each step zeroes the GDN state slots (in
    every layer) of exactly the requests it admits: their rows."""
    case("scheduler admissions zero their GDN state slots")
    from muserve_amd.state_pool import StatePool
    rng = np.random.default_rng(5)
    batch = 6
    cache = PagedKVCache(256, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    pool = StatePool(num_layers=3, num_slots=batch + 2, state_shape=(2, 16, 16),
                     conv_shape=(64, 4), device=DEV)
    s = ContinuousBatchScheduler(max_batch_size=batch, max_seq_len=512, kv_cache=cache,
                                 chunked_prefill_size=96, state_pool=pool)
    for i in range(14):
        s.add_request(req(i, int(rng.integers(1, 120)), int(rng.integers(1, 6))))
    admitted_total = 0
    while True:
        pool.state.fill_(7.0)  # every slot dirty before the step
        pool.conv.fill_(3.0)
        plan = s.plan_step()
        if plan is None:
            break
        torch.cuda.synchronize()
        rows = {r.row for r in plan.admitted}
        assert rows == set(plan.rows.cpu().tolist()[plan.num_entries - len(plan.admitted):])
        st, cv = pool.state.cpu(), pool.conv.cpu().float()
        for slot in range(pool.num_slots):
            want = 0.0 if slot in rows else None
            if want is None:
                assert (st[:, slot] == 7.0).all() and (cv[:, slot] == 3.0).all()
            else:
                assert (st[:, slot] == 0).all() and (cv[:, slot] == 0).all()
        admitted_total += len(rows)
        s.complete_step(plan)
    pool.check_errors()
    assert admitted_total == 14
