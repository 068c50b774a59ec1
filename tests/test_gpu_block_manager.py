"""GPU block manager (mkv_bm_step) vs the OrderedDict model, request by request:
status, hits, page tables, copy-on-write pairs, eviction order, and the final
free stack / LRU order / refcounts / cached hashes; plus the copied pages."""
import numpy as np
import pytest
import torch

import bench
from muserve_amd import _lib
from muserve_amd.block_manager import BlockManager
from muserve_amd.kv_cache import PagedKVCache
from muserve_amd.prefix_hash import as_u64, page_hashes
from oracle.blocks import OK, OOM, BlockManagerModel
from oracle.sha import page_hashes as cpu_page_hashes
from tests.gpu_util import DEV, bits16, case

pytestmark = pytest.mark.gpu


def interleaved_ops(n, batch):
    """Per batch: admit the batch, then release the previous batch's requests
    one at a time between them (single releases, not runs)."""
    out = []
    for b0 in range(0, n, batch):
        prev = list(range(max(0, b0 - batch), b0))
        cur = list(range(b0, min(n, b0 + batch)))
        ops = []
        for i, r in enumerate(cur):
            ops.append(r)
            if i < len(prev):
                ops.append(-(prev[i] + 1))
        ops += [-(r + 1) for r in prev[len(cur):]]
        out.append(ops)
    return out


def serving_ops(seed, cap=16):
    """The serving scheduler's pattern: per step the releases of a few finished
    requests (often one; now and then half of them), then new admits while
    fewer than cap are live."""
    def ops_fn(n, batch):
        rng = np.random.default_rng(seed)
        live, out, nxt = [], [], 0
        while nxt < n or live:
            k = int(rng.integers(0, 4)) if rng.random() < 0.7 else len(live) // 2
            k = min(len(live), k) if nxt < n else len(live)
            idx = sorted(rng.choice(len(live), size=k, replace=False).tolist(), reverse=True)
            rel = [live.pop(i) for i in idx]
            room = max(0, cap - len(live))
            new = list(range(nxt, min(n, nxt + min(room, int(rng.integers(0, batch + 1))))))
            nxt += len(new)
            live += new
            out.append([-(r + 1) for r in rel] + new)
        return out
    return ops_fn


def random_ops(seed):
    """Random op streams: per step a leading run of 0..all releases of live
    requests (random order), then new admits shuffled with more releases."""
    def ops_fn(n, batch):
        rng = np.random.default_rng(seed)
        live, out, nxt = [], [], 0
        while nxt < n or live:
            rng.shuffle(live)
            k = int(rng.integers(0, len(live) + 1))
            lead, live = live[:k], live[k:]
            m = int(rng.integers(0, len(live) + 1))
            tail_rel, live = live[:m], live[m:]
            new = list(range(nxt, min(n, nxt + int(rng.integers(1, 2 * batch)))))
            nxt += len(new)
            rest = new + [-(r + 1) for r in tail_rel]
            rng.shuffle(rest)
            ops = [-(r + 1) for r in lead] + rest
            if ops:
                out.append(ops)
            live += new
        return out
    return ops_fn


def synthetic_keys(n, seed, alphabet, max_pages, skew):
    """Prefix keys over a small alphabet instead of SHA-256: key i mixes key
    i-1 with symbol i (SplitMix64 finaliser), so equal keys mean equal
    prefixes, as for page hashes. Symbols are drawn geometrically (parameter
    `skew`), so requests of one step share prefixes of many lengths; the
    rarest first symbol gives the key 0. Half the requests start with a prefix
    of an earlier one."""
    rng = np.random.default_rng(seed)
    M = (1 << 64) - 1

    def mix(prev, sym):
        z = (prev * 0x9E3779B97F4A7C15 + sym + 1) & M
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)
    lens, keys = [], []
    for r in range(n):
        nt = int(rng.integers(1, max_pages * 16 + 1))
        m = nt // 16
        sym = np.minimum(rng.geometric(skew, m) - 1, alphabet - 1)
        if r and rng.random() < 0.5:
            src = keys[int(rng.integers(0, r))]
            c = int(rng.integers(0, min(len(src), m) + 1))
        else:
            src, c = [], 0
        k = list(src[:c])
        for i in range(c, m):
            k.append(0 if i == 0 and sym[i] == alphabet - 1 else
                     mix(k[-1] if i else 0x5EED, int(sym[i])))
        lens.append(nt)
        keys.append(k)
    return lens, [np.array(k, dtype=np.uint64).view(np.int64) for k in keys]


def run(P, n, batch, seed, n_templates, template_len, suffix, width, with_data=False,
        ops_fn=bench.prefix_ops, keys=None, split=False, data_layers=2):
    """Drives the manager through ops_fn's steps and checks it against the
    model; returns the statuses, the model and the final snapshot. `keys` =
    (token counts, per-request key lists) replaces the hashed prompts.
    split: each step as step_begin + step_end; where the committed-admit
    count grew by the step's admits, their results read between the halves
    are checked too (snap["early_steps"] counts those steps).
    with_data: a bf16 pool of data_layers layers holds random pages and each
    step's copy-on-write pairs are copied by the library. The expected pool
    applies the model's pairs (torch indexing: on the CPU for small pools, on
    the device for large ones), and every page of the pool is compared at the
    end."""
    if keys is None:
        reqs = bench.prefix_requests(n, seed=seed, n_templates=n_templates,
                                     template_len=template_len, suffix=suffix)
        lens = [len(x) for x in reqs]
        cu = np.concatenate([[0], np.cumsum(lens)])
        flat = torch.from_numpy(np.concatenate(reqs)).to(DEV)
        hashes, cu_pages = page_hashes(flat, cu)
        hu = as_u64(hashes)
        for r in range(n):  # every request's GPU page hashes are its hashlib prefix keys
            assert hu[cu_pages[r]:cu_pages[r + 1]].tolist() == cpu_page_hashes(reqs[r]), r
    else:
        lens, kl = keys
        cu_pages = np.concatenate([[0], np.cumsum([len(k) for k in kl])]).astype(np.int64)
        flat = np.concatenate([np.asarray(k, dtype=np.int64) for k in kl] + [np.zeros(0, np.int64)])
        hashes = torch.from_numpy(flat).to(DEV)
        hu = as_u64(hashes)
    free = np.random.default_rng(seed).permutation(P).tolist()
    bm = BlockManager(P, n, width, DEV, free_order=free, evict_log_capacity=1 << 20)
    model = BlockManagerModel(P, free)
    cache = cpu = None
    if with_data:
        cache = PagedKVCache(P, num_layers=data_layers, dtype=torch.bfloat16, device=DEV,
                             verbose=False)
        if data_layers <= 2:
            cpu = torch.randn(cache.cache.shape,
                              generator=torch.Generator().manual_seed(seed)).bfloat16()
            cache.cache.copy_(cpu.to(DEV))
        else:  # a full-size pool: random pages made on the device, the expected pool too
            cache.cache.normal_(generator=torch.Generator(device=DEV).manual_seed(seed))
            cpu = cache.cache.clone()
    off = torch.from_numpy(cu_pages).to(DEV)
    ntok = torch.tensor(lens, dtype=torch.int32, device=DEV)
    want = {}
    early_steps = cow_pairs = 0
    for ops in ops_fn(n, batch):
        admits = [o for o in ops if o >= 0]  # consecutive request ids
        mid = None
        if split:
            before = int(bm.spec_done_word().item())
            bm.step_begin(torch.tensor(ops, dtype=torch.int32), hashes, off, ntok)
            if admits and int(bm.spec_done_word().item()) - before == len(admits):
                mid = (bm.status.cpu().tolist(), bm.hits.cpu().tolist(), bm.tables.cpu())
            bm.step_end()
        else:
            bm.step(torch.tensor(ops, dtype=torch.int32), hashes, off, ntok)
        pairs = []
        for op in ops:
            if op >= 0:
                h = [int(v) for v in hu[cu_pages[op]:cu_pages[op + 1]]]
                want[op] = model.admit(op, h, lens[op])
                if want[op]["cow_src"] >= 0:
                    pairs.append((want[op]["cow_src"], want[op]["cow_dst"]))
            elif -op - 1 in model.reqs:
                model.release(-op - 1)
        if mid is not None:  # every admit's result was final after the first half
            early_steps += 1
            for op in admits:
                assert mid[0][op] == want[op]["status"], op
                if want[op]["status"] == OK:
                    assert mid[1][op] == want[op]["hits"], op
                    assert mid[2][op, :-(-lens[op] // 16)].tolist() == want[op]["table"], op
        if with_data and admits:
            bm.copy_on_write(cache, min(admits), min(admits) + len(admits))
            if pairs:  # a fresh destination is never another pair's source
                src = torch.tensor([p[0] for p in pairs], device=cpu.device)
                dst = torch.tensor([p[1] for p in pairs], device=cpu.device)
                cpu[:, :, dst] = cpu[:, :, src]
            cow_pairs += len(pairs)
    bm.check_errors()
    ctr = bm.counters()
    print(f"speculation: {ctr[7]} admits resolved, {ctr[8]} left to the sequential kernels",
          flush=True)
    status = bm.status.cpu().tolist()
    hits, cl = bm.hits.cpu().tolist(), bm.child_last.cpu().tolist()
    cs, cd = bm.cow_src.cpu().tolist(), bm.cow_dst.cpu().tolist()
    tables = bm.tables.cpu()
    for r in range(n):
        w = want[r]
        released = status[r] == 3
        assert (OK if released else status[r]) == w["status"], r
        if w["status"] != OK:
            continue
        assert hits[r] == w["hits"], r
        npg = -(-lens[r] // 16)
        assert tables[r, :npg].tolist() == w["table"], r
        assert (cl[r], cs[r], cd[r]) == (w["child_last"], w["cow_src"], w["cow_dst"]), r
    snap = bm.snapshot()
    assert snap["table_ok"]  # entries = cached pages, with their keys and refcounts
    assert snap["tombs_ok"]  # the tombstone count matches the table
    assert snap["last_ok"] and snap["evictable"] == len(snap["lru"])
    assert snap["free"] == model.free
    assert snap["lru"] == model.lru_order()
    assert snap["ref"] == model.ref
    assert snap["hash"] == model.hash
    log = bm.evict_log.cpu().tolist()[:snap["log_len"]]
    assert log == model.evicted
    if with_data:
        if cpu.device.type == "cpu":
            assert torch.equal(bits16(cache.cache), cpu.view(torch.int16))
        else:
            assert torch.equal(cache.cache.view(torch.int16), cpu.view(torch.int16))
        cache.check_errors()
    # read-only probe of every request against the final table
    pages, hit = bm.probe(hashes, off)
    pages, hit = pages.cpu().tolist(), hit.cpu().tolist()
    bm.check_errors()
    for r in range(n):
        h = [int(v) for v in hu[cu_pages[r]:cu_pages[r + 1]]]
        want_pages = [model.table.get(x, -1) for x in h]
        assert pages[cu_pages[r]:cu_pages[r + 1]] == want_pages, r
        lead = next((i for i, p in enumerate(want_pages) if p < 0), len(h))
        assert hit[r] == lead, r
    assert bm.snapshot()["lru"] == snap["lru"]  # nothing moved
    snap["early_steps"] = early_steps
    snap["cow_pairs"] = cow_pairs
    return status, model, snap


def test_small_pool_evictions_oom_and_cow():
    case("block manager: 72-page pool, 240 requests, batches of 6")
    status, model, snap = run(P=72, n=240, batch=6, seed=104, n_templates=6, template_len=128,
                        suffix=(1, 120), width=32, with_data=True)
    assert OOM in status and len(model.evicted) > 100
    # OOMs and same-step evictions of hit pages send admits to the sequential
    # kernels; the rest are resolved by the many-CU speculation
    assert snap["spec_done"] > 0 and snap["spec_left"] > 0


def test_larger_trace_with_ring_compaction():
    case("block manager: 3000-page pool, 1200 requests, batches of 32")
    status, model, snap = run(P=3000, n=1200, batch=32, seed=7, n_templates=24, template_len=512,
                        suffix=(16, 600), width=96)
    assert len(model.evicted) > 1000


def test_long_requests_past_the_register_held_pages():
    # up to 2600 pages per request: pages past the first 1024 of a request take
    # the kernel's memory-resident path (probe, pin, register)
    case("block manager: 5400-page pool, 14 requests of ~2300-2600 pages")
    status, model, snap = run(P=5400, n=14, batch=2, seed=11, n_templates=2, template_len=36000,
                        suffix=(1, 5000), width=2600)
    assert len(model.evicted) > 500


def test_many_evictions_rebuild_the_table():
    # 72 pages and a 4096-slot table: ~10,800 evictions leave tombstones past
    # a quarter of the table many times over, so the table is rebuilt repeatedly
    case("block manager: 72-page pool, 1500 requests, batches of 6")
    status, model, snap = run(P=72, n=1500, batch=6, seed=21, n_templates=40, template_len=128,
                        suffix=(1, 120), width=32)
    assert len(model.evicted) > 2000


def test_long_release_runs():
    # batches of 100 requests of ~190-230 pages: runs of 100 releases dropping
    # ~21,000 page references, in a pool small enough to evict thousands
    case("block manager: 4000-page pool, 400 requests, batches of 100")
    status, model, snap = run(P=4000, n=400, batch=100, seed=9, n_templates=8, template_len=3000,
                        suffix=(1, 600), width=240)
    assert len(model.evicted) > 4000


def test_release_run_past_the_reference_limit():
    # 1000 releases of ~1102 pages each drop ~1.1M references: the many-CU
    # release run stops at the op boundary below 2^20 and the one-workgroup
    # step kernel releases the rest
    case("block manager: 5000-page pool, 2000 requests of ~1102 pages, batches of 1000")
    status, model, snap = run(P=5000, n=2000, batch=1000, seed=17, n_templates=1, template_len=17600,
                        suffix=(1, 20), width=1102)
    assert OOM not in status


@pytest.mark.parametrize("seed", [31, 32, 33])
def test_random_release_runs_and_interleavings(seed):
    case(f"block manager: random op streams, 96-page pool, seed {seed}")
    status, model, snap = run(P=96, n=400, batch=8, seed=seed, n_templates=5, template_len=160,
                        suffix=(1, 100), width=32, with_data=seed == 31,
                        ops_fn=random_ops(seed))
    assert len(model.evicted) > 100


@pytest.mark.parametrize("seed,ops", [(61, "serving"), (62, "random")])
def test_step_in_two_halves(seed, ops):
    # step_begin + step_end is step. Steps of at most 8 ops run on the step
    # kernel alone (in step_end); in longer ones a single leading release goes
    # through the release run, so the admits after it are resolved on many CUs,
    # and where every admit was committed by the first half its results are
    # final there
    case(f"block manager: step_begin + step_end, {ops} ops, seed {seed}")
    fn = serving_ops(seed) if ops == "serving" else random_ops(seed)
    steps = fn(240, 16)
    assert sum(len(o) > 8 for o in steps) > 10
    assert ops != "serving" or sum(len(o) <= 8 for o in steps) > 20
    status, model, snap = run(P=192, n=240, batch=16, seed=seed, n_templates=6, template_len=128,
                              suffix=(1, 120), width=32, ops_fn=fn, split=True)
    if ops == "serving":  # (the CPU model admits every request of 21 long steps)
        assert snap["early_steps"] > 10
    assert len(model.evicted) > 50


def test_single_releases_between_admits():
    case("block manager: 72-page pool, 240 requests, releases between admits")
    status, model, snap = run(P=72, n=240, batch=6, seed=105, n_templates=6, template_len=128,
                        suffix=(1, 120), width=32, ops_fn=interleaved_ops)
    assert len(model.evicted) > 100


@pytest.mark.parametrize("seed,P,batch,alphabet,skew,ops", [
    (41, 96, 12, 16, 0.3, "random"),   # ~380 evictions, ~40 OOMs
    (42, 300, 48, 16, 0.3, "batch"),   # ~1850 evictions
    (43, 1000, 160, 32, 0.2, "batch"),  # ~6600 evictions
])
def test_prefix_keys_over_a_small_alphabet(seed, P, batch, alphabet, skew, ops):
    # prefixes shared at every length inside one step (hits on pages that
    # earlier admits of the step register), and the key 0: the many-CU
    # resolution must resolve each admit exactly or hand it to the
    # sequential kernels
    case(f"block manager: recurring synthetic keys, {P}-page pool, batches of {batch}, "
         f"alphabet {alphabet}, seed {seed}")
    n = 12 * batch
    status, model, snap = run(P=P, n=n, batch=batch, seed=seed, n_templates=0, template_len=0,
                              suffix=None, width=12,
                              keys=synthetic_keys(n, seed, alphabet, 12, skew),
                              ops_fn=random_ops(seed) if ops == "random" else bench.prefix_ops)
    assert len(model.evicted) > 200 and snap["spec_done"] > 0 and snap["spec_left"] > 0


@pytest.mark.parametrize("seed,P,batch,alphabet,skew,ops,n", [
    (48, 9000, 1500, 32, 0.2, "batch", 3000),        # 1500 admits a step: past the 1024 speculated
    (49, 300, 40, 16, 0.3, "interleaved", 480),      # releases between the admits
    (50, 4000, 600, 64, 0.1, "random", 1800),        # release runs, ~320 OOMs, ~2400 evictions
    (51, 700, 200, 8, 0.4, "batch", 1200),           # ~400 OOMs in a tight pool
])
def test_speculation_edges_against_the_model(seed, P, batch, alphabet, skew, ops, n):
    case(f"block manager: prefix keys, {P}-page pool, {n} requests, batches of {batch}, "
         f"{ops} op order, seed {seed}")
    fn = {"batch": bench.prefix_ops, "interleaved": interleaved_ops,
          "random": random_ops(seed)}[ops]
    status, model, snap = run(P=P, n=n, batch=batch, seed=seed, n_templates=0, template_len=0,
                              suffix=None, width=12,
                              keys=synthetic_keys(n, seed, alphabet, 12, skew), ops_fn=fn)
    assert snap["spec_done"] > 0
    if batch > 1024:  # the admits past the first 1024 of a step are the group kernel's
        assert snap["spec_done"] + snap["spec_left"] < n


def test_requests_of_up_to_2048_pages_resolved_together():
    # prompts of 16,000-token templates plus up to 16,000 more tokens (1,000 to
    # ~1,970 pages): every admit fits the speculation's 2048 positions, and the
    # pool is small enough for thousands of evictions
    case("block manager: 24,000-page pool, 60 requests of 1000-1971 pages, batches of 12")
    status, model, snap = run(P=24000, n=60, batch=12, seed=46, n_templates=3, template_len=16000,
                              suffix=(1, 16000), width=1971)
    assert len(model.evicted) > 5000
    assert snap["spec_done"] > 30


def test_eviction_wave_longer_than_the_lru_window():
    # step 1 admits 512 requests of 512 fresh pages (262,144 pages cached once
    # step 2 releases them); step 3 admits 400 more, whose 204,800 takes evict
    # ~167k pages: more than the speculation's 131,072-entry LRU window, so
    # the admit that runs past it and every later one go to the sequential
    # kernels
    case("block manager: 300,000-page pool, an eviction wave of ~167k pages in one step")
    n, m = 912, 512
    rng = np.random.default_rng(44)
    keys = [rng.integers(1, 1 << 63, m, dtype=np.int64) for _ in range(n)]
    lens = [16 * m] * n
    steps = [list(range(512)), [-(r + 1) for r in range(512)], list(range(512, n))]
    status, model, snap = run(P=300_000, n=n, batch=0, seed=44, n_templates=0, template_len=0,
                              suffix=None, width=m, keys=(lens, keys),
                              ops_fn=lambda n_, b_: steps)
    assert len(model.evicted) > 131_072
    assert snap["spec_done"] >= 512 and snap["spec_left"] > 0


def test_request_admitted_twice_in_one_step():
    # the speculation stops before a request's second admit in a step; the
    # sequential kernels admit it again (the model overwrites its tables)
    case("block manager: a request admitted twice in one step")
    lens, keys = synthetic_keys(6, 45, 4, 6, 0.5)
    steps = [[0, 1, 0, 2], [-1, -2, -3, 3, 4], [-4, -5, 5, 5]]
    status, model, snap = run(P=64, n=6, batch=0, seed=45, n_templates=0, template_len=0,
                              suffix=None, width=6, keys=(lens, keys),
                              ops_fn=lambda n_, b_: steps)
    admits = sum(op >= 0 for st in steps for op in st)
    assert snap["spec_done"] < admits  # the repeats (and what follows) went sequential


def test_duplicate_release_is_flagged_once():
    case("block manager: a request released twice in one step")
    reqs = bench.prefix_requests(3, seed=3, n_templates=1, template_len=64, suffix=(5, 20))
    lens = [len(x) for x in reqs]
    cu = np.concatenate([[0], np.cumsum(lens)])
    hashes, cu_pages = page_hashes(torch.from_numpy(np.concatenate(reqs)).to(DEV), cu)
    off = torch.from_numpy(cu_pages).to(DEV)
    ntok = torch.tensor(lens, dtype=torch.int32, device=DEV)
    free = list(range(64))
    bm = BlockManager(64, 3, 8, DEV, free_order=free)
    model = BlockManagerModel(64, free)
    bm.step(torch.tensor([0, 1, 2], dtype=torch.int32), hashes, off, ntok)
    hu = as_u64(hashes)
    for r in range(3):
        model.admit(r, [int(v) for v in hu[cu_pages[r]:cu_pages[r + 1]]], lens[r])
    bm.step(torch.tensor([-1, -2, -1, -3], dtype=torch.int32), hashes, off, ntok)  # 0 twice
    with pytest.raises(_lib.MkvDeviceError, match="block manager"):
        bm.check_errors()
    for r in (0, 1, 2):
        model.release(r)
    snap = bm.snapshot()
    assert snap["table_ok"] and snap["last_ok"]
    assert snap["ref"] == model.ref and snap["free"] == model.free
    assert snap["lru"] == model.lru_order()


def test_release_of_unknown_request_is_flagged():
    case("block manager: release of a request never admitted")
    bm = BlockManager(64, 4, 8, DEV)
    z = torch.zeros(5, dtype=torch.int64, device=DEV)
    bm.step(torch.tensor([-(2 + 1)], dtype=torch.int32), z[:0], z, torch.zeros(4, dtype=torch.int32))
    with pytest.raises(_lib.MkvDeviceError, match="block manager"):
        bm.check_errors()
    # (check_errors cleared the word) the same inside a leading run of releases
    bm.step(torch.tensor([-(2 + 1), -(1 + 1)], dtype=torch.int32), z[:0], z,
            torch.zeros(4, dtype=torch.int32))
    with pytest.raises(_lib.MkvDeviceError, match="block manager"):
        bm.check_errors()
    assert bm.snapshot()["last_ok"]
