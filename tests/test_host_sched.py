"""Host half of the product scheduler (reference protocol and the paged step's
decisions and page allocation) against the scheduler oracle, on the CPU: the
pool lives on the CPU and only metadata runs."""
import numpy as np
import pytest

from muserve_amd.kv_cache import PagedKVCache
from muserve_amd.scheduler import ContinuousBatchScheduler, InferenceRequest, RequestState
from oracle import paged as pg
from oracle import sched as S
from tests.test_oracle_sched import known_chunked_trace

ENTRY = 8


def cpu_cache(n, free=None):
    c = PagedKVCache(n, num_layers=1, device="cpu", verbose=False)
    if free is not None:
        c._free_pages = list(free)
    return c


def req(rid, n, gen=256):
    return InferenceRequest(request_id=rid, input_ids=list(range(n)), max_new_tokens=gen)


def test_reference_protocol_known_trace():
    """The same hand trace as the oracle's (muserve/scheduler.py:73-111)."""
    s = ContinuousBatchScheduler(max_batch_size=2)
    a, b, c = req("a", 4), req("b", 4), req("c", 4)
    for r in (a, b, c):
        s.add_request(r)
    pre, dec = s.schedule_step()
    assert [r.request_id for r in pre] == ["a", "b"] and dec == []
    assert a.state == RequestState.PREFILLING and c.state == RequestState.WAITING
    s.finish_prefill(pre)
    assert a.first_token_at is not None and s.num_running == 2 and s.num_waiting == 1
    pre, dec = s.schedule_step()
    assert pre == [] and [r.request_id for r in dec] == ["a", "b"]
    s.finish_request(a)
    assert a.is_done and a.finished_at is not None
    pre, dec = s.schedule_step()
    assert [r.request_id for r in pre] == ["c"] and [r.request_id for r in dec] == ["b"]
    s.finish_prefill(pre)
    pre, dec = s.schedule_step()
    assert pre == [] and [r.request_id for r in dec] == ["b", "c"]
    assert not s.is_idle


def as_oracle_step(s: ContinuousBatchScheduler, plan):
    """The product's host plan in the oracle's step format; slots and tables
    from the sequences' page tables after the step (what the kernel reads)."""
    if plan is None:
        return {"rids": [], "kinds": [], "starts": [], "counts": [], "rows": [], "slots": [],
                "positions": [], "cu_seqlens": [0], "lens": [], "tables": []}
    n = plan.num_entries
    ent = plan.upload[:n * ENTRY].reshape(n, ENTRY)
    out = {"rids": [r.request_id for r in plan.entries],
           "kinds": ["decode"] * plan.num_decode + ["prefill"] * len(plan.prefill),
           "starts": ent[:, 1].tolist(), "counts": ent[:, 2].tolist(),
           "rows": ent[:, 0].tolist(), "slots": [], "positions": [], "cu_seqlens": [0],
           "lens": [], "tables": []}
    for i, r in enumerate(plan.entries):
        t = r.seq.page_table
        start, count = int(ent[i, 1]), int(ent[i, 2])
        assert int(ent[i, 6]) == out["cu_seqlens"][-1]
        out["cu_seqlens"].append(out["cu_seqlens"][-1] + count)
        out["positions"] += list(range(start, start + count))
        out["slots"] += [t[p // 16] * 16 + p % 16 for p in range(start, start + count)]
        out["lens"].append(start + count)
        out["tables"].append(list(t) + [0] * (s.width - len(t)))
        # the new pages the upload carries are the tail of the page table
        held, new, off = int(ent[i, 3]), int(ent[i, 4]), int(ent[i, 5])
        assert list(plan.upload[n * ENTRY + off:n * ENTRY + off + new]) == t[held:held + new]
    return out


def test_product_known_chunked_trace():
    cache = cpu_cache(8)
    s = ContinuousBatchScheduler(max_batch_size=4, max_seq_len=64, kv_cache=cache,
                                 chunked_prefill_size=20)
    for rid, n in (("a", 30), ("b", 10)):
        s.add_request(req(rid, n, gen=2))
    state = {}

    def step():
        state["plan"] = s.plan_host()
        return as_oracle_step(s, state["plan"])

    def complete():
        s.complete_step(state["plan"])

    known_chunked_trace(step, complete)
    assert cache._free_pages == [0, 1, 2, 3, 4, 7, 6, 5]
    assert s.is_idle


@pytest.mark.parametrize("seed,pages,chunk,batch", [(0, 40, 48, 6), (1, 40, 48, 6),
                                                    (2, 64, 100, 4), (3, 400, 4096, 16),
                                                    (4, 24, 33, 8)])
def test_product_matches_oracle_random(seed, pages, chunk, batch):
    rng = np.random.default_rng(seed)
    free = rng.permutation(pages).tolist()
    pool = pg.PoolModel(pages, free)
    m = S.ChunkedSchedulerModel(batch, chunk, pool, 256, eos=7)
    cache = cpu_cache(pages, free)
    s = ContinuousBatchScheduler(max_batch_size=batch, max_seq_len=256, kv_cache=cache,
                                 chunked_prefill_size=chunk, eos_token_id=7)
    specs = [(i, int(rng.integers(1, 160)), int(rng.integers(1, 40))) for i in range(40)]
    pending = list(specs)
    oracle_oom = product_oom = None
    for step in range(3000):
        while pending and rng.random() < 0.3:
            i, n, g = pending.pop(0)
            m.add(S.Req(i, n, g))
            s.add_request(req(i, n, g))
        try:
            want = m.step()
        except RuntimeError as e:
            oracle_oom = str(e)
        try:
            plan = s.plan_host()
        except RuntimeError as e:
            product_oom = str(e)
        if oracle_oom or product_oom:
            assert oracle_oom and product_oom and "KV cache OOM" in product_oom
            return
        got = as_oracle_step(s, plan)
        assert got == want, f"step {step}"
        assert cache._free_pages == pool.free
        toks = rng.integers(0, 64, len(want["rids"])).tolist()
        m.complete(toks)
        if plan is not None:
            s.complete_step(plan, toks)
        if not pending and s.is_idle:
            break
    assert not m.running and not m.prefilling and not m.waiting
    assert sorted(cache._free_pages) == list(range(pages))


def test_product_oom_when_decode_finds_no_page():
    cache = cpu_cache(2)
    s = ContinuousBatchScheduler(max_batch_size=2, max_seq_len=64, kv_cache=cache,
                                 chunked_prefill_size=64)
    s.add_request(req("a", 16))
    s.add_request(req("b", 16))
    p = s.plan_host()                 # both prompts fill one page each
    assert [r.request_id for r, _, _ in p.prefill] == ["a", "b"]
    s.complete_step(p)
    with pytest.raises(RuntimeError, match="KV cache OOM"):
        s.plan_host()                 # each decode needs a second page


def test_chunk_waits_for_pages_and_request_stays_queued():
    cache = cpu_cache(1)
    s = ContinuousBatchScheduler(max_batch_size=4, max_seq_len=64, kv_cache=cache,
                                 chunked_prefill_size=64)
    s.add_request(req("a", 20, gen=1))
    s.add_request(req("b", 5, gen=1))
    p = s.plan_host()                 # a takes the only page: 16 of its 20 tokens
    assert [(r.request_id, st, n) for r, st, n in p.prefill] == [("a", 0, 16)]
    assert s.num_waiting == 1 and s.num_prefilling == 1
    s.complete_step(p)
    assert s.plan_host() is None      # a needs a page; b waits behind it
    assert s.num_waiting == 1


def test_argument_errors():
    cache = cpu_cache(8)
    s = ContinuousBatchScheduler(max_batch_size=2, max_seq_len=32, kv_cache=cache)
    with pytest.raises(ValueError, match="empty prompt"):
        s.add_request(req("e", 0))
    with pytest.raises(ValueError, match="exceeds max_seq_len"):
        s.add_request(req("l", 33))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        s.plan_step()
    s.add_request(req("a", 4))
    p = s.plan_host()
    with pytest.raises(RuntimeError, match="complete_step"):
        s.plan_host()
    with pytest.raises(ValueError, match="tokens for"):
        s.complete_step(p, [1, 2])


def test_max_seq_len_finishes_a_request():
    cache = cpu_cache(8)
    s = ContinuousBatchScheduler(max_batch_size=2, max_seq_len=18, kv_cache=cache,
                                 chunked_prefill_size=64)
    r = req("a", 16, gen=100)
    s.add_request(r)
    for _ in range(3):
        p = s.plan_host()
        s.complete_step(p)
    # prompt 16, then decodes at positions 16 and 17; the cache is full at 18
    assert r.is_done and r.seq.seq_len == 18 and len(r.generated_tokens) == 3


def test_prefix_reuse_with_gdn_states_is_rejected():
    """A prefix hit skips prefill of its pages, but GDN states are not cached
    with the pages: a scheduler with both a state pool and a block manager
    would run the recurrent layers from zero states mid-prompt."""
    from types import SimpleNamespace

    from muserve_amd.scheduler import ContinuousBatchScheduler
    with pytest.raises(ValueError, match="does not cache GDN states"):
        ContinuousBatchScheduler(max_batch_size=4, state_pool=SimpleNamespace(num_slots=8),
                                 block_manager=object())


def test_block_manager_step_refuses_a_pending_half_step():
    from muserve_amd.block_manager import BlockManager
    bm = BlockManager.__new__(BlockManager)  # no device state: the guard comes first
    bm._pending = ((), ())
    with pytest.raises(RuntimeError, match="awaits its step_end"):
        bm.step(None, None, None, None)
