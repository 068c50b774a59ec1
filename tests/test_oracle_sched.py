"""The scheduler oracle against the reference scheduler's behaviour
(muserve/scheduler.py:73-123, traced by hand) and against invariants of the
paged step (CPU only)."""
import numpy as np
import pytest

from oracle import paged as pg
from oracle import sched as S


def test_reference_schedule_known_trace():
    """schedule_step / finish_prefill / finish_request of muserve/scheduler.py:73-111
    with max_batch_size 2 and three requests, traced by hand."""
    s = S.ReferenceScheduler(max_batch_size=2)
    a, b, c = S.Req("a", 4), S.Req("b", 4), S.Req("c", 4)
    for r in (a, b, c):
        s.add_request(r)
    pre, dec = s.schedule_step()
    assert [r.rid for r in pre] == ["a", "b"] and dec == []
    assert a.state == S.PREFILLING and c.state == S.WAITING
    s.finish_prefill(pre)
    pre, dec = s.schedule_step()          # batch full: nothing admitted
    assert pre == [] and [r.rid for r in dec] == ["a", "b"]
    s.finish_request(a)
    pre, dec = s.schedule_step()          # a dropped, c admitted
    assert [r.rid for r in pre] == ["c"] and [r.rid for r in dec] == ["b"]
    s.finish_prefill(pre)
    pre, dec = s.schedule_step()
    assert pre == [] and [r.rid for r in dec] == ["b", "c"]


def known_chunked_trace(impl_step, impl_complete):
    """chunk 20, pool of 8 pages with free list [0..7], prompts of 30 and 10
    tokens, 2 new tokens each — every slot derived by hand from the LIFO list
    (pages 7, 6 to the first request, 5 to the second)."""
    steps = []
    steps.append(impl_step())
    impl_complete()
    steps.append(impl_step())
    impl_complete()
    steps.append(impl_step())
    impl_complete()
    steps.append(impl_step())
    s1, s2, s3, s4 = steps
    assert s1["rids"] == ["a"] and s1["starts"] == [0] and s1["counts"] == [20]
    assert s1["slots"] == list(range(112, 128)) + list(range(96, 100))
    assert s1["rows"] == [0] and s1["cu_seqlens"] == [0, 20] and s1["lens"] == [20]
    assert s1["tables"][0][:3] == [7, 6, 0]
    assert s2["rids"] == ["a", "b"] and s2["kinds"] == ["prefill", "prefill"]
    assert s2["starts"] == [20, 0] and s2["counts"] == [10, 10]
    assert s2["slots"] == list(range(100, 110)) + list(range(80, 90))
    assert s2["rows"] == [0, 1] and s2["cu_seqlens"] == [0, 10, 20] and s2["lens"] == [30, 10]
    assert s3["kinds"] == ["decode", "decode"] and s3["slots"] == [110, 90]
    assert s3["positions"] == [30, 10]
    assert s4["rids"] == []
    return steps


def test_oracle_known_chunked_trace():
    pool = pg.PoolModel(8)
    m = S.ChunkedSchedulerModel(max_batch_size=4, chunk=20, pool=pool, max_seq_len=64)
    for rid, n in (("a", 30), ("b", 10)):
        m.add(S.Req(rid, n, max_new_tokens=2))
    known_chunked_trace(m.step, m.complete)
    # retired in running order: a's pages [7, 6], then b's [5]
    assert pool.free == [0, 1, 2, 3, 4, 7, 6, 5]


def test_oracle_reduces_to_reference_admission():
    """With an unbounded budget and pool, the paged step admits exactly the
    requests the reference's schedule_step would, in the same order."""
    rng = np.random.default_rng(5)
    ref = S.ReferenceScheduler(max_batch_size=3)
    m = S.ChunkedSchedulerModel(3, 10**9, pg.PoolModel(4096), 1 << 14)
    reqs = [(f"r{i}", int(rng.integers(1, 40)), int(rng.integers(1, 5))) for i in range(9)]
    model_req = {}
    for rid, n, g in reqs:
        ref.add_request(S.Req(rid, n, g))
        model_req[rid] = S.Req(rid, n, g)
        m.add(model_req[rid])
    for _ in range(40):
        pre, dec = ref.schedule_step()
        out = m.step()
        kinds = dict(zip(out["rids"], out["kinds"]))
        assert [r.rid for r in dec] == [k for k, v in kinds.items() if v == "decode"]
        assert [r.rid for r in pre] == [k for k, v in kinds.items() if v == "prefill"]
        ref.finish_prefill(pre)
        m.complete()
        for r in ref.running:   # the reference's caller finishes what the model finished
            if model_req[r.rid].state == S.FINISHED:
                ref.finish_request(r)
        if not ref.running and not ref.waiting:
            break
    assert not ref.running and not ref.waiting and not m.waiting


def run_random(seed, max_batch=6, chunk=48, pages=40, max_seq_len=200, n_req=30):
    rng = np.random.default_rng(seed)
    free = rng.permutation(pages).tolist()
    pool = pg.PoolModel(pages, free)
    m = S.ChunkedSchedulerModel(max_batch, chunk, pool, max_seq_len)
    reqs = [S.Req(i, int(rng.integers(1, 120)), int(rng.integers(1, 30))) for i in range(n_req)]
    return rng, pool, m, reqs


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_invariants(seed):
    rng, pool, m, reqs = run_random(seed)
    pending = list(reqs)
    for step in range(2000):
        while pending and rng.random() < 0.3:
            m.add(pending.pop(0))
        try:
            out = m.step()
        except RuntimeError as e:     # decode found no page: the reference's OOM
            assert "KV cache OOM" in str(e)
            return
        held = [p for r in m.running + m.prefilling for p in r.seq.page_table]
        assert sorted(held + pool.free) == list(range(pool.num_free + len(held)))
        assert len(set(held)) == len(held)
        assert sum(c for c, k in zip(out["counts"], out["kinds"]) if k == "prefill") <= m.chunk
        assert len(set(out["slots"])) == len(out["slots"])
        assert len(set(out["rows"])) == len(out["rows"])
        assert all(0 <= r < m.max_batch_size for r in out["rows"])
        # every slot is the page-table position of its token (brute force)
        for i, rid in enumerate(out["rids"]):
            t = out["tables"][i]
            for j in range(out["cu_seqlens"][i], out["cu_seqlens"][i + 1]):
                p = out["positions"][j]
                assert out["slots"][j] == t[p // 16] * 16 + p % 16
            assert out["lens"][i] == out["starts"][i] + out["counts"][i]
        m.complete(list(rng.integers(0, 100, len(out["rids"]))))
        if not pending and not m.waiting and not m.running and not m.prefilling:
            break
    assert all(r.state == S.FINISHED for r in reqs)
    assert sorted(pool.free) == list(range(40))


# ---- prefix reuse through the block manager (PrefixSchedulerModel) ----

from oracle.blocks import BlockManagerModel  # noqa: E402


def _prefix_model(chunk=40, B=4, bm_pages=8, private=(8, 16), max_seq_len=128):
    pool = pg.PoolModel(private[1], list(range(*private)))
    return S.PrefixSchedulerModel(B, chunk, BlockManagerModel(bm_pages), pool, max_seq_len)


def test_prefix_model_known_trace():
    """Worked out by hand: A = T + 5 tokens and B = T + 3 tokens share a
    48-token template T (3 shareable pages each), C has 10 tokens of its own.
    Budget 40 per step, block-manager pages 0..7 (popped 7, 6, 5, ...),
    private pages 8..15 (popped 15, 14, ...)."""
    T = list(range(1000, 1048))
    A = S.PReq("A", T + [1, 2, 3, 4, 5], max_new_tokens=2)
    Bq = S.PReq("B", T + [6, 7, 8], max_new_tokens=2)
    C = S.PReq("C", list(range(2000, 2010)), max_new_tokens=2)
    m = _prefix_model()
    for r in (A, Bq, C):
        m.add(r)
    # step 1: A is the only candidate (40 - 53 < 0 ends the candidates); its
    # three template pages are fresh (7, 6, 5), its tail page 15; 40 tokens
    s1 = m.step()
    assert s1["ops"] == [0] and s1["admitted"] == [("A", 0, 0)] and s1["skipped"] == 0
    assert s1["counts"] == [40] and s1["starts"] == [0]
    assert s1["slots"] == list(range(112, 128)) + list(range(96, 112)) + list(range(80, 88))
    m.complete()
    # step 2: A's last 13 tokens (page 5's second half, tail page 15), then B
    # hits all three template pages: 48 tokens skipped, its 3 tokens go to its
    # tail page 14
    s2 = m.step()
    assert s2["ops"] == [1] and s2["admitted"] == [("B", 1, 3)] and s2["skipped"] == 48
    assert s2["rids"] == ["A", "B"] and s2["starts"] == [40, 48] and s2["counts"] == [13, 3]
    assert s2["slots"] == list(range(88, 96)) + list(range(240, 245)) + [224, 225, 226]
    assert s2["tables"][1][:4] == [7, 6, 5, 14]
    assert m.complete() == []
    # step 3: A and B decode in their tail pages; C (no shareable page, no
    # block-manager op) prefills into page 13
    s3 = m.step()
    assert s3["ops"] == [] and s3["kinds"] == ["decode", "decode", "prefill"]
    assert s3["slots"] == [245, 227] + list(range(208, 218))
    assert {r.rid for r in m.complete()} == {"A", "B"}
    # step 4: A and B release their pages in retire order; the template pages
    # reach refcount 0 with B's release, tail first: LRU 5, 6, 7
    s4 = m.step()
    assert s4["ops"] == [-1, -2] and s4["slots"] == [218]
    assert m.bm.lru_order() == [5, 6, 7]
    assert m.pool.free == [8, 9, 10, 11, 12, 15, 14]
    assert m.skipped == 48
    m.bm.check_invariants()


def _random_prompts(rng, n, lo, hi, vocab=151936):
    return [rng.integers(0, vocab, int(rng.integers(lo, hi))).tolist() for _ in range(n)]


@pytest.mark.parametrize("seed", [0, 1])
def test_prefix_model_reduces_to_chunked_without_sharing(seed):
    """With no prompt prefix in common and pools that never run out, prefix
    reuse changes nothing in the schedule: the same entries (request, kind,
    start, count, row) step for step as ChunkedSchedulerModel."""
    rng = np.random.default_rng(seed)
    prompts = _random_prompts(rng, 60, 1, 300)
    outs = rng.integers(1, 40, 60)
    pm = S.PrefixSchedulerModel(8, 128, BlockManagerModel(100000),
                                pg.PoolModel(200000, list(range(100000, 200000))), 4096)
    cm = S.ChunkedSchedulerModel(8, 128, pg.PoolModel(100000), 4096)
    for i, (p, o) in enumerate(zip(prompts, outs)):
        pm.add(S.PReq(i, p, int(o)))
        cm.add(S.Req(i, len(p), int(o)))
    for _ in range(2000):
        a, b = pm.step(), cm.step()
        key = ("rids", "kinds", "starts", "counts", "rows", "lens")
        assert {k: a[k] for k in key} == {k: b[k] for k in key}
        assert a["skipped"] == 0
        pm.complete()
        cm.complete()
        if not (pm.waiting or pm.running or pm.prefilling):
            break
    assert not (cm.waiting or cm.running or cm.prefilling)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_prefix_model_invariants_on_shared_prompts(seed):
    """Zipf-shared templates with small pools (evictions, a block manager that
    turns candidates away, private pages running short): block-manager
    invariants after every step, every slot of a step distinct and inside its
    request's pages, the private pages partitioned between the list and the
    live requests, and no hit page read before it is written (the model
    asserts it)."""
    rng = np.random.default_rng(seed)
    templates = [rng.integers(0, 151936, 96).tolist() for _ in range(4)]
    zipf = 1.0 / np.arange(1, 5) ** 1.1
    prompts = []
    for _ in range(80):
        t = templates[rng.choice(4, p=zipf / zipf.sum())]
        prompts.append(t[:int(rng.integers(20, 97))] + rng.integers(0, 151936,
                                                                    int(rng.integers(0, 40))).tolist())
    m = S.PrefixSchedulerModel(6, 64, BlockManagerModel(40),
                               pg.PoolModel(80, list(range(40, 80))), 512)
    reqs = [S.PReq(i, p, int(rng.integers(1, 30))) for i, p in enumerate(prompts)]
    for r in reqs:
        m.add(r)
    for _ in range(5000):
        s = m.step()
        m.bm.check_invariants()
        assert len(set(s["slots"])) == len(s["slots"])
        live = m.running + m.prefilling
        private_held = [p for r in live for p in r.seq.page_table[r.fb:]]
        assert sorted(private_held + m.pool.free) == list(range(40, 80))
        assert all(p < 40 for r in live for p in r.seq.page_table[:r.fb])
        m.complete()
        if not (m.waiting or m.running or m.prefilling):
            break
    assert all(r.state == S.FINISHED for r in reqs)
    assert m.skipped > 0 and m.bm.evicted
