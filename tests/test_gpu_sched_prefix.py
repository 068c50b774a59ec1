"""Prefix reuse in the serving step: ContinuousBatchScheduler with a
BlockManager (GPU page hashes, mkv_bm_step admissions and releases, the
chunked prefill starting at the first uncached page) against
oracle.sched.PrefixSchedulerModel, which composes the chunked scheduler with
oracle.blocks.BlockManagerModel: every step's slots, positions, cu_seqlens,
tables, lengths, rows and block-manager ops, the prompt tokens skipped, and
at the end the eviction order and the block manager's free stack and LRU."""
import numpy as np
import pytest
import torch

from muserve_amd.block_manager import BlockManager
from muserve_amd.kernels import attention as A
from muserve_amd.kv_cache import PagedKVCache
from muserve_amd.scheduler import ContinuousBatchScheduler, InferenceRequest
from oracle import attention as oatt
from oracle import paged as pg
from oracle import sched as S
from oracle.blocks import BlockManagerModel
from tests.gpu_util import DEV, case
from tests.test_gpu_attention import within_one_ulp
from tests.test_gpu_sched import check_plan

pytestmark = pytest.mark.gpu


def zipf_prompts(rng, n, n_templates, template_len, suffix, vocab=151936, s=1.1):
    templates = rng.integers(0, vocab, (n_templates, template_len))
    w = 1.0 / np.arange(1, n_templates + 1) ** s
    out = []
    for _ in range(n):
        t = templates[rng.choice(n_templates, p=w / w.sum())]
        cut = int(rng.integers(template_len // 2, template_len + 1))
        out.append(t[:cut].tolist() + rng.integers(0, vocab, int(rng.integers(*suffix))).tolist())
    return out


@pytest.mark.parametrize("seed,bm_pages,private,chunk,batch,max_seq", [
    (0, 64, 64, 96, 6, 512),        # small pools: evictions, the last candidate turned away
    (1, 400, 300, 512, 16, 1024),
    (2, 3000, 2000, 4096, 64, 4096),
])
def test_prefix_scheduler_matches_model(seed, bm_pages, private, chunk, batch, max_seq):
    case(f"prefix-reuse scheduler seed {seed}: block-manager pages {bm_pages}, private "
         f"{private}, chunk {chunk}, batch {batch}")
    rng = np.random.default_rng(seed)
    prompts = zipf_prompts(rng, 6 * batch, 6, max_seq // 3, (1, max_seq // 8))
    outs = rng.integers(1, 40, len(prompts))
    P = bm_pages + private
    bm_free = rng.permutation(bm_pages).tolist()
    cache = PagedKVCache(P, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    width = -(-max_seq // 16)
    bm = BlockManager(bm_pages, 2 * batch, width, DEV, free_order=bm_free,
                      evict_log_capacity=1 << 16)
    s = ContinuousBatchScheduler(max_batch_size=batch, max_seq_len=max_seq, kv_cache=cache,
                                 chunked_prefill_size=chunk, eos_token_id=3, block_manager=bm)
    # the private list: the cache's pages past the block manager's, in its order
    private_free = list(cache._free_pages)
    assert sorted(private_free) == list(range(bm_pages, P))
    m = S.PrefixSchedulerModel(batch, chunk, BlockManagerModel(bm_pages, bm_free),
                               pg.PoolModel(P, private_free), max_seq, eos=3)
    pending = list(range(len(prompts)))
    steps = skipped = 0
    for step in range(20000):
        while pending and rng.random() < 0.4:
            i = pending.pop(0)
            m.add(S.PReq(i, prompts[i], int(outs[i])))
            s.add_request(InferenceRequest(request_id=i, input_ids=prompts[i],
                                           max_new_tokens=int(outs[i])))
        want = m.step()
        plan = s.plan_step()
        check_plan(s, plan, want, step)
        if plan is not None:
            assert plan.bm_ops == want["ops"], f"step {step}: block-manager ops"
            assert plan.skipped_tokens == want["skipped"], f"step {step}: skipped tokens"
            skipped += plan.skipped_tokens
        else:
            assert want["skipped"] == 0
        toks = rng.integers(0, 64, len(want["rids"])).tolist()
        m.complete(toks)
        if plan is not None:
            s.complete_step(plan, toks)
            steps += 1
        if not pending and s.is_idle:
            break
    s.check_errors()
    assert not pending and s.is_idle and steps > 20
    assert skipped == m.skipped > 0 and s.prefix_skipped == skipped
    # rounds read after the many-CU half (every admit committed there) and
    # after the one-workgroup kernels (short rounds, turn-aways)
    print(f"block-manager rounds read early {s.bm_early_rounds}, late {s.bm_late_rounds}",
          flush=True)
    # the block manager's state equals the model's: eviction order, free
    # stack, LRU order, refcounts (every request released)
    snap = bm.snapshot()
    nlog = snap["log_len"]
    assert bm.evict_log[:nlog].cpu().tolist() == m.bm.evicted
    assert snap["free"] == m.bm.free
    assert snap["lru"] == m.bm.lru_order()
    assert snap["ref"] == m.bm.ref and snap["table_ok"]
    if seed == 0:
        assert m.bm.evicted, "the small case is meant to evict"


def _kv(ids: torch.Tensor, pos: torch.Tensor, salt: float) -> torch.Tensor:
    """K (or V) of a token as a function of its id and position only (host,
    float32 then bf16): a prefix shared by two prompts has equal K/V in both,
    as in a real model."""
    d = torch.arange(256, dtype=torch.float32)
    x = ids.to(torch.float32)[:, None] * 0.37 + pos.to(torch.float32)[:, None] * 0.011 + d * salt
    return torch.sin(x).bfloat16()[:, None, :]


def test_prefix_pages_hold_every_sequence_kv():
    """Serving steps with prefix reuse writing real K/V: after every step's
    append, every entry's sequence gathered through its block table (shared
    cached pages, its own tail and decode pages) equals the K/V of its own
    tokens at their positions, bit for bit; and the step's decode attention
    over those tables, with the block manager's pages as shared_pages (read
    through the caches, the sequences' spans sorted by first page), is within
    the oracle's tolerance."""
    case("prefix-reuse scheduler drives appends; every sequence gathered back each step")
    rng = np.random.default_rng(7)
    batch, max_seq, chunk, bm_pages, private = 6, 512, 96, 64, 64
    prompts = zipf_prompts(rng, 30, 4, 160, (1, 40))
    cache = PagedKVCache(bm_pages + private, num_layers=1, dtype=torch.bfloat16, device=DEV,
                         verbose=False)
    bm = BlockManager(bm_pages, 2 * batch, -(-max_seq // 16), DEV,
                      free_order=rng.permutation(bm_pages).tolist())
    s = ContinuousBatchScheduler(max_batch_size=batch, max_seq_len=max_seq, kv_cache=cache,
                                 chunked_prefill_size=chunk, eos_token_id=3, block_manager=bm)
    reqs = [InferenceRequest(request_id=i, input_ids=p, max_new_tokens=int(rng.integers(1, 30)))
            for i, p in enumerate(prompts)]
    for r in reqs:
        s.add_request(r)
    checked = attn_checked = 0
    for step in range(5000):
        plan = s.plan_step()
        if plan is None:
            if s.is_idle:
                break
            continue
        ids, pos = [], []
        for r, (_, start, count) in zip(plan.entries, [(None, r_.seq.seq_len - 1, 1)
                                                        for r_ in plan.decode] + plan.prefill):
            seq = r.input_ids + r.generated_tokens
            ids += seq[start:start + count]
            pos += range(start, start + count)
        ids_t, pos_t = torch.tensor(ids), torch.tensor(pos)
        assert plan.positions.cpu().tolist() == pos
        cache.append(plan.slot_mapping, _kv(ids_t, pos_t, 0.1).to(DEV),
                     _kv(ids_t, pos_t, 0.07).to(DEV), layer=0)
        lens = plan.seq_lens.cpu().numpy().astype(np.int64)
        cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=DEV)
        kg, vg = cache.gather(0, plan.block_tables, plan.seq_lens, out_len=int(lens.max()),
                              cu_out=cu)
        want_ids = torch.tensor([t for r, n in zip(plan.entries, lens)
                                 for t in (r.input_ids + r.generated_tokens)[:n]])
        want_pos = torch.cat([torch.arange(n) for n in lens])
        assert torch.equal(kg.cpu().view(torch.int16),
                           _kv(want_ids, want_pos, 0.1).view(torch.int16)), f"step {step}"
        assert torch.equal(vg.cpu().view(torch.int16),
                           _kv(want_ids, want_pos, 0.07).view(torch.int16)), f"step {step}"
        checked += len(lens)
        nd = plan.num_decode
        if nd:
            q = torch.from_numpy(rng.standard_normal((nd, 1, 4, 256)).astype(np.float32))
            q = q.bfloat16().to(DEV)
            kc, vc = cache.get_kv_by_layer(0)
            out = A.attn_decode(q, kc, vc, plan.seq_lens[:nd], plan.block_tables[:nd],
                                shared_pages=bm.num_pages)
            torch.cuda.synchronize()
            A.check_errors(DEV)
            want = oatt.decode_attention(q[:, 0].float().cpu().numpy(),
                                         kc.float().cpu().numpy(), vc.float().cpu().numpy(),
                                         lens[:nd], plan.block_tables[:nd].cpu().numpy(),
                                         256 ** -0.5, stats=True)
            within_one_ulp(out[:, 0], want)
            attn_checked += 1
        s.complete_step(plan, rng.integers(0, 64, plan.num_entries).tolist())
    s.check_errors()
    cache.check_errors()
    assert s.is_idle and s.prefix_skipped > 0 and checked > 100 and attn_checked > 20
