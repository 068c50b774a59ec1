"""Parity at the benchmark configurations' full sizes, through properties that
do not depend on size: append -> gather round trips, oracle checks of sampled
rows, gather/scatter identities, and the whole prefix-cache trace against the
OrderedDict model."""
import numpy as np
import pytest
import torch

import bench
from muserve_amd.kv_cache import PagedKVCache, SequenceKVState, prefill_slot_mapping, reserve_tokens, slot_mapping_for
from muserve_amd.state_pool import StatePool
from oracle import fp8 as ref
from tests.gpu_util import DEV, case
from tests.test_gpu_block_manager import run as run_block_manager

pytestmark = pytest.mark.gpu


def _tables(seqs, width):
    bt = torch.zeros(len(seqs), width, dtype=torch.int32)
    for b, s in enumerate(seqs):
        bt[b, :len(s.page_table)] = torch.tensor(s.page_table, dtype=torch.int32)
    return bt.to(DEV)


def test_decode_config_append_gather_round_trip():
    case("full size: 256 sequences, lognormal lengths (seed 102), 15 layers, padded gather")
    ctx = bench.context_lengths()
    B, L = len(ctx), 15
    cache = PagedKVCache(int(np.sum(-(-ctx // 16))) + 16, num_layers=L, dtype=torch.bfloat16,
                         device=DEV, verbose=False)
    cache.shuffle_free_list(torch.Generator().manual_seed(102))
    seqs = [SequenceKVState() for _ in range(B)]
    slots = prefill_slot_mapping(cache, seqs, ctx.tolist())
    T = int(ctx.sum())
    bt = _tables(seqs, max(len(s.page_table) for s in seqs))
    lens = torch.from_numpy(ctx.astype(np.int32)).to(DEV)
    lpad = int(-(-int(ctx.max()) // 16) * 16)
    # row of padded output [B*lpad] for every appended token, in append order
    rows = np.concatenate([b * lpad + np.arange(n) for b, n in enumerate(ctx)])
    rows = torch.from_numpy(rows).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(102)
    for layer in range(L):
        k = torch.randn(T, 1, 256, generator=gen, device=DEV).bfloat16()
        v = torch.randn(T, 1, 256, generator=gen, device=DEV).bfloat16()
        cache.append(slots, k, v, layer=layer)
        kd, vd = cache.gather(layer, bt, lens, out_len=lpad)
        for got, src in ((kd, k), (vd, v)):
            want = torch.zeros(B * lpad, 1, 256, dtype=torch.bfloat16, device=DEV)
            want[rows] = src
            assert torch.equal(got.reshape(B * lpad, 1, 256).view(torch.int16),
                               want.view(torch.int16)), layer
        del kd, vd
    cache.check_errors()


def test_fp8_config_append_and_window_against_oracle():
    case("full size: fp8 pool of 262160 pages x 15 layers, 32 x 2048-token chunks into 128k contexts")
    R, CHUNK, CTX, WIN, L = 32, 2048, 131072, 8192, 15
    cache = PagedKVCache(R * CTX // 16 + 16, num_layers=L, dtype=torch.float8_e4m3fn, device=DEV,
                         verbose=False)
    cache.shuffle_free_list(torch.Generator().manual_seed(103))
    seqs = [SequenceKVState() for _ in range(R)]
    prior = CTX - CHUNK
    gen = torch.Generator(device=DEV).manual_seed(103)

    def kv(t):
        x = torch.randn(L, t, 1, 256, generator=gen, device=DEV)
        boost = torch.rand(L, t, 1, 256, generator=gen, device=DEV) < 0.01
        return torch.where(boost, x * 20.0, x).bfloat16()

    # positions before the window's start are reserved (pages allocated) but
    # never read; the window's prior tokens and the chunk are appended
    fill = WIN - CHUNK
    for s in seqs:
        reserve_tokens(cache, s, prior - fill)
    sl = torch.from_numpy(np.concatenate(
        [slot_mapping_for(s, reserve_tokens(cache, s, fill), fill) for s in seqs])).to(DEV)
    cache.append(sl, kv(len(sl)), kv(len(sl)))
    chunk_slots = torch.from_numpy(np.concatenate(
        [slot_mapping_for(s, reserve_tokens(cache, s, CHUNK), CHUNK) for s in seqs])).to(DEV)
    k, v = kv(R * CHUNK), kv(R * CHUNK)
    cache.append(chunk_slots, k, v)
    cache.check_errors()
    # every appended row of every layer vs the oracle's quantiser (codes and
    # scales, bit for bit)
    for layer in range(L):
        for kvi, x in ((0, k), (1, v)):
            q, sc = ref.quantize_rows(x[layer].cpu())
            got_q = cache.cache[layer, kvi].view(torch.uint8).reshape(-1, 1, 256)[chunk_slots].cpu()
            got_s = cache.scales[layer, kvi].reshape(-1, 1)[chunk_slots].cpu()
            assert torch.equal(got_q, q), (layer, kvi)
            assert torch.equal(got_s.view(torch.int32), sc.view(torch.int32)), (layer, kvi)
    # dequant-gather of every request's last 8192 tokens in every layer vs the
    # oracle's dequantisation of the pool rows the tables name
    bt = _tables(seqs, CTX // 16)
    lens = torch.full((R,), CTX, dtype=torch.int32, device=DEV)
    starts = lens - WIN
    cu = torch.arange(R + 1, dtype=torch.int64, device=DEV) * WIN
    pos = torch.arange(CTX - WIN, CTX, device=DEV)
    slot = (bt.to(torch.int64)[:, pos // 16] * 16 + pos % 16).reshape(-1)  # [R * WIN]
    for layer in range(L):
        kd, vd = cache.gather(layer, bt, lens, out_len=WIN, starts=starts, cu_out=cu)
        for kvi, got in ((0, kd), (1, vd)):
            codes = cache.cache[layer, kvi].view(torch.uint8).reshape(-1, 1, 256)[slot].cpu()
            scales = cache.scales[layer, kvi].reshape(-1, 1)[slot].cpu()
            want = ref.dequant_rows(codes, scales)
            assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16)), (layer, kvi)
    cache.check_errors()


@pytest.mark.timeout(600)
def test_decode_config_steps_against_oracle():
    """The decode configuration's step sequence at full size: 256 sequences
    (lognormal lengths, seed 102), 15 layers, 3 steps of device slot
    assignment (pages taken at page boundaries from a shuffled free list),
    all-layer appends and padded gathers of the grown tables. Per step: the
    slots equal the oracle's decode_step, the device tables and lengths equal
    the oracle's; the appended rows sit at the oracle's slots; every layer's
    padded gather equals torch's index_select of the same rows on the device,
    and its first and last sequences equal the CPU oracle's gather; at the end
    an int64 checksum of each layer's pool equals the one before the steps
    with the overwritten rows swapped for the appended ones (nothing else
    was written)."""
    from muserve_amd.kv_cache import BlockTables
    from oracle import paged as pref

    B, L, STEPS = 256, 15, 3
    ctx = bench.context_lengths()
    case(f"full size: {STEPS} decode steps, batch {B}, {L} layers, ctx sum {int(ctx.sum())}")
    pages = int(np.sum(-(-(ctx + STEPS) // 16))) + 64
    cache = PagedKVCache(pages, num_layers=L, dtype=torch.bfloat16, device=DEV, verbose=False)
    gen = torch.Generator(device=DEV).manual_seed(102)
    for l in range(L):
        cache.cache[l].normal_(generator=gen)
    cache.shuffle_free_list(torch.Generator().manual_seed(102))
    pm = pref.PoolModel(pages, list(cache._free_pages))
    seqs = [SequenceKVState() for _ in range(B)]
    oseqs = [pref.SeqModel() for _ in range(B)]
    for s_, o_, n in zip(seqs, oseqs, ctx):
        reserve_tokens(cache, s_, int(n))
        o_.add_tokens(pm, int(n))
    width = int(-(-(int(ctx.max()) + STEPS) // 16))
    bt = BlockTables(cache, seqs, max_pages=width)

    def checksum(l):
        return int(cache.cache[l].view(torch.int16).sum(dtype=torch.int64))

    before = [checksum(l) for l in range(L)]
    delta = [0] * L
    for step in range(STEPS):
        slots = bt.decode_step()
        want = pref.decode_step(pm, oseqs)
        assert slots.cpu().tolist() == want, f"step {step}: slots"
        otab = torch.zeros(B, width, dtype=torch.int32)
        for b, o in enumerate(oseqs):
            otab[b, :len(o.page_table)] = torch.tensor(o.page_table, dtype=torch.int32)
        olens = torch.tensor([o.seq_len for o in oseqs], dtype=torch.int32)
        assert torch.equal(bt.tables.cpu(), otab) and torch.equal(bt.seq_lens.cpu(), olens)
        kn = torch.randn(L, B, 1, 256, generator=gen, device=DEV).bfloat16()
        vn = torch.randn(L, B, 1, 256, generator=gen, device=DEV).bfloat16()
        idx = torch.tensor(want, dtype=torch.int64, device=DEV)
        for l in range(L):
            old = cache.cache[l].reshape(2, -1, 256)[:, idx]
            delta[l] -= int(old.view(torch.int16).sum(dtype=torch.int64))
        cache.append(slots, kn, vn)
        for l in range(L):
            new = cache.cache[l].reshape(2, -1, 256)[:, idx]
            assert torch.equal(new[0].view(torch.int16), kn[l, :, 0].view(torch.int16)), (step, l)
            assert torch.equal(new[1].view(torch.int16), vn[l, :, 0].view(torch.int16)), (step, l)
            delta[l] += int(new.view(torch.int16).sum(dtype=torch.int64))
        W = bt.padded_len()
        pos = torch.arange(W, device=DEV)
        valid = pos[None, :] < bt.seq_lens.to(torch.int64)[:, None]  # [B, W]
        rows = (bt.tables.to(torch.int64)[:, (pos // 16).clamp(max=width - 1)] * 16 + pos % 16)
        rows = torch.where(valid, rows, torch.zeros_like(rows))
        for l in range(L):
            kd, vd = cache.gather(l, bt.tables, bt.seq_lens, out_len=W)
            for kvi, got in ((0, kd), (1, vd)):
                plane = cache.cache[l, kvi].reshape(-1, 256)
                ref_out = plane.index_select(0, rows.reshape(-1)).reshape(B, W, 256)
                ref_out = torch.where(valid[..., None], ref_out, torch.zeros_like(ref_out))
                assert torch.equal(got[:, :, 0].view(torch.int16), ref_out.view(torch.int16)), \
                    (step, l, kvi)
                if l in (0, L - 1):  # the CPU oracle on the first and the last sequence
                    for b in (0, B - 1):
                        cpu_plane = cache.cache[l, kvi][otab[b, :len(oseqs[b].page_table)]
                                                        .to(DEV).to(torch.int64)].cpu()
                        t = torch.arange(len(oseqs[b].page_table), dtype=torch.int32)[None]
                        w = pref.gather_padded(cpu_plane, t, olens[b:b + 1], W)
                        assert torch.equal(got[b].cpu().view(torch.int16),
                                           w[0].view(torch.int16)), (step, l, kvi, b)
            del kd, vd
    cache.check_errors()
    assert [checksum(l) for l in range(L)] == [b + d for b, d in zip(before, delta)]


def test_gdn_config_gather_scatter_identities():
    case("full size: GDN pool 45 x 1024 slots x ([8,128,128] fp32 + [2048,4] bf16), batch 256")
    S, G, B = 1024, 45, 256
    pool = StatePool(num_layers=G, num_slots=S, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(105)
    pool.state.normal_(generator=gen)
    pool.conv.normal_(generator=gen)
    slots = torch.randperm(S, generator=torch.Generator().manual_seed(105))[:B]
    idx = slots.to(DEV)
    s32 = idx.to(torch.int32)
    for g in range(G):
        before_s, before_c = pool.state[g].clone(), pool.conv[g].clone()
        st, cv = pool.gather(g, s32)
        assert torch.equal(st, before_s[idx]) and torch.equal(cv, before_c[idx]), g
        pool.scatter(g, s32, st + 1.0, cv + 1.0)
        want_s, want_c = before_s, before_c
        want_s[idx] = st + 1.0
        want_c[idx] = cv + 1.0
        assert torch.equal(pool.state[g], want_s) and torch.equal(pool.conv[g], want_c), g
    pool.check_errors()


@pytest.mark.timeout(900)
def test_prefix_config_full_trace_against_model():
    # 4096 requests (Zipf(1.1) over 64 templates of 4096 ids + 64..1024-token
    # suffixes), batches of 256, 65536 pages: every request's page hashes
    # against hashlib, every admit, table, hit count, copy-on-write pair, the
    # 89k-entry eviction order and the final state; the copies run on a real
    # 15-layer bf16 pool of 65536 pages (16 GB of random pages), compared page
    # for page at the end with the model's pairs applied to a copy of it
    case("full size: prefix cache, 4096 requests, 65536 pages x 15 layers, batches of 256")
    status, model, snap = run_block_manager(P=65536, n=4096, batch=256, seed=104, n_templates=64,
                                      template_len=4096, suffix=(64, 1024), width=320,
                                      with_data=True, data_layers=15)
    assert len(model.evicted) > 50000
    assert snap["spec_done"] + snap["spec_left"] == 4096  # every admit was speculated
    assert snap["cow_pairs"] > 3000  # copy-on-write pairs copied and checked


@pytest.mark.timeout(600)
def test_gdn_config_interleaved_with_decode_appends_against_oracle():
    """The hybrid decode step at full size, 60 layers in model order for 3
    steps: every attention layer (l % 4 == 3, muserve/memory/kv_cache.py:20)
    appends the step's decode token of 256 sequences (slots from the device
    decode step, lognormal contexts, seed 102), every GDN layer gathers the
    256 requests' recurrent + conv states from the 1024-slot pools, updates
    them (x * 0.5 + layer, conv + step) and scatters them back. The CPU oracle
    does the same on copies of both state pools and of the KV pool; at the end
    all three pools are compared byte for byte."""
    from muserve_amd.kv_cache import BlockTables
    from muserve_amd.state_pool import gdn_ordinal
    from oracle import paged as pref
    from oracle import state as sref

    S, G, B, L, STEPS = 1024, 45, 256, 15, 3
    case(f"full size: 60 layers in model order x {STEPS} steps, GDN pools 45 x 1024 slots, "
         f"decode appends on 15 layers, batch {B}")
    pool = StatePool(num_layers=G, num_slots=S, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(105)
    pool.state.normal_(generator=gen)
    pool.conv.normal_(generator=gen)
    cpu_state = torch.empty(pool.state.shape, dtype=pool.state.dtype)
    cpu_conv = pool.conv.cpu()
    for g in range(G):
        cpu_state[g].copy_(pool.state[g])
    slots = torch.randperm(S, generator=torch.Generator().manual_seed(105))[:B].to(torch.int32)
    slots_d = slots.to(DEV)

    ctx = bench.context_lengths()
    pages = int(np.sum(-(-(ctx + STEPS) // 16))) + 64
    cache = PagedKVCache(pages, num_layers=L, dtype=torch.bfloat16, device=DEV, verbose=False)
    cache.shuffle_free_list(torch.Generator().manual_seed(102))
    pmodel = pref.PoolModel(pages, list(cache._free_pages))
    seqs = [SequenceKVState() for _ in range(B)]
    oseqs = [pref.SeqModel() for _ in range(B)]
    for s_, o_, n in zip(seqs, oseqs, ctx):
        reserve_tokens(cache, s_, int(n))
        o_.add_tokens(pmodel, int(n))
    bt = BlockTables(cache, seqs, max_pages=int(-(-(int(ctx.max()) + STEPS) // 16)))
    cpu_kv = torch.zeros(cache.cache.shape, dtype=torch.bfloat16)
    kg = torch.Generator().manual_seed(5)

    for step in range(STEPS):
        kv_slots = bt.decode_step()
        want_slots = pref.decode_step(pmodel, oseqs)
        assert kv_slots.cpu().tolist() == want_slots, f"step {step}"
        want_slots = torch.tensor(want_slots)
        for layer in range(60):
            if layer % 4 == 3:
                a = layer // 4
                k = torch.randn(B, 1, 256, generator=kg).bfloat16()
                v = torch.randn(B, 1, 256, generator=kg).bfloat16()
                cache.append(kv_slots, k.to(DEV), v.to(DEV), layer=a)
                pref.append(cpu_kv, want_slots, k, v, layer=a)
                continue
            g = gdn_ordinal(layer)
            st, cv = pool.gather(g, slots_d)
            st.mul_(0.5).add_(float(g + 1))
            cv.add_(float(step + 1))
            pool.scatter(g, slots_d, st, cv)
            ost = sref.gather(cpu_state, g, slots)
            ocv = sref.gather(cpu_conv, g, slots)
            ost.mul_(0.5).add_(float(g + 1))
            ocv.add_(float(step + 1))
            sref.scatter(cpu_state, g, slots, ost)
            sref.scatter(cpu_conv, g, slots, ocv)
    torch.cuda.synchronize()
    pool.check_errors()
    cache.check_errors()
    for g in range(G):
        assert torch.equal(pool.state[g].cpu().view(torch.int32), cpu_state[g].view(torch.int32)), g
    assert torch.equal(pool.conv.cpu().view(torch.int16), cpu_conv.view(torch.int16))
    for a in range(L):
        assert torch.equal(cache.cache[a].cpu().view(torch.int16), cpu_kv[a].view(torch.int16)), a
    assert [s.page_table for s in seqs] == [s.page_table for s in oseqs]
