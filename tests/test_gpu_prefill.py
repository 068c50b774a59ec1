"""GPU parity of the varlen prefill attention (attn_prefill over contiguous
K/V, attn_prefill_paged over the pool) vs the float64 oracle.

Tolerance, per output element: one bf16 ulp of the float64 value plus
2^-8 x the attended mass sum_j p_j |v_j| / sum_j p_j. The second term covers
the probabilities' rounding to bf16 for the P V product (relative 2^-9 each,
as in flash attention's bf16 path) with a factor of 2 for the fp32
evaluation."""
import numpy as np
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.kernels import attention as A
from muserve_amd.kv_cache import PagedKVCache
from muserve_amd.scheduler import ContinuousBatchScheduler, InferenceRequest
from oracle import attention as att
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


def within(got: torch.Tensor, want) -> None:
    want, mass = want
    got = got.float().cpu().numpy().astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    tol = ulp + 2.0 ** -8 * mass
    err = np.abs(got - want)
    bad = err > tol
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements out of tolerance; worst "
                           f"{err[bad].max()} at {np.argwhere(bad)[0]}")


def seqs(lens, seed):
    g = torch.Generator().manual_seed(seed)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    return g, cu


@pytest.mark.parametrize("causal", [True, False])
def test_contiguous_varlen_matches_oracle(causal):
    lens = [1, 5, 15, 16, 17, 31, 33, 64, 100, 257, 600]
    case(f"attn_prefill contiguous varlen causal={causal} lens {lens}")
    g, cu = seqs(lens, 31 + causal)
    T = int(cu[-1])
    q = torch.randn(T, 4, 256, generator=g).bfloat16()
    k = torch.randn(T, 1, 256, generator=g).bfloat16()
    v = torch.randn(T, 1, 256, generator=g).bfloat16()
    out = A.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), max(lens),
                         max(lens), causal=causal)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.prefill_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                 cu.numpy(), 256 ** -0.5, causal, cu_k=cu.numpy(), stats=True)
    within(out, want)


def test_many_sequences_without_key_splits():
    """64 sequences of 256 queries fill 512 workgroups: one key range each,
    the output written by the attention kernel itself."""
    case("attn_prefill 64 x 256 tokens (no key splits)")
    lens = [256] * 64
    g, cu = seqs(lens, 33)
    T = int(cu[-1])
    q = torch.randn(T, 4, 256, generator=g).bfloat16()
    k = torch.randn(T, 1, 256, generator=g).bfloat16()
    v = torch.randn(T, 1, 256, generator=g).bfloat16()
    out = A.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), 256, 256)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    sample = 4  # the oracle on the first sequences (each is independent)
    n = 256 * sample
    want = att.prefill_attention(q[:n].float().numpy(), k[:n].float().numpy(),
                                 v[:n].float().numpy(), cu[:sample + 1].numpy(), 256 ** -0.5, True,
                                 cu_k=cu[:sample + 1].numpy(), stats=True)
    within(out[:n], want)


def test_contiguous_with_prefix_two_kv_heads_and_scale():
    """nk > nq (a prefix before the queries), 2 KV heads (8 query heads), a
    softmax scale of 0.1, and a sequence with more queries than keys."""
    lq = [7, 40, 3, 129]
    lk = [20, 40, 1, 300]
    case(f"attn_prefill with prefix: nq {lq}, nk {lk}, 2 KV heads")
    g = torch.Generator().manual_seed(35)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), 8, 256, generator=g).bfloat16()
    k = torch.randn(int(cu_k[-1]), 2, 256, generator=g).bfloat16()
    v = torch.randn(int(cu_k[-1]), 2, 256, generator=g).bfloat16()
    out = A.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV), max(lq),
                         max(lk), softmax_scale=0.1)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.prefill_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                 cu_q.numpy(), 0.1, True, cu_k=cu_k.numpy(), stats=True)
    within(out, want)
    assert not out[int(cu_q[2]):int(cu_q[2]) + 2].float().abs().sum().item()  # saw nothing


def test_paged_chunks_match_oracle():
    """Chunked prefill over the pool: each sequence has a cached prefix and a
    chunk (appended first); queries are the chunk's tokens."""
    prefix = [0, 3, 16, 100, 1000]
    chunk = [17, 1, 32, 64, 300]
    case(f"attn_prefill_paged prefix {prefix} chunk {chunk}")
    g = torch.Generator().manual_seed(36)
    P = 256
    kc = torch.randn(P, 16, 1, 256, generator=g).bfloat16()
    vc = torch.randn(P, 16, 1, 256, generator=g).bfloat16()
    perm = torch.randperm(P, generator=g)
    lens = [p + c for p, c in zip(prefix, chunk)]
    width = max(-(-n // 16) for n in lens)
    table = torch.zeros(len(lens), width, dtype=torch.int32)
    at = 0
    for b, n in enumerate(lens):
        m = -(-n // 16)
        table[b, :m] = perm[at:at + m].to(torch.int32)
        at += m
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(chunk)]), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), 4, 256, generator=g).bfloat16()
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    out = A.attn_prefill_paged(q.to(DEV), kc.to(DEV), vc.to(DEV), cu_q.to(DEV), seq_lens.to(DEV),
                               table.to(DEV), max(chunk))
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.prefill_attention(q.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                 cu_q.numpy(), 256 ** -0.5, True, lens_k=seq_lens.numpy(),
                                 page_table=table.numpy(), stats=True)
    within(out, want)


def test_scheduler_prefill_entries_through_the_pool():
    """A scheduler step's prefill entries: their tokens' K/V appended through
    plan.slot_mapping, then attn_prefill_paged on plan.cu_seqlens /
    plan.seq_lens / plan.block_tables past the decode entries."""
    case("scheduler prefill chunks -> append -> attn_prefill_paged")
    rng = np.random.default_rng(7)
    g = torch.Generator(device=DEV).manual_seed(7)
    cache = PagedKVCache(1024, num_layers=1, dtype=torch.bfloat16, device=DEV, verbose=False)
    cache._free_pages = rng.permutation(1024).tolist()
    s = ContinuousBatchScheduler(max_batch_size=6, max_seq_len=2048, kv_cache=cache,
                                 chunked_prefill_size=300)
    for i in range(8):
        s.add_request(InferenceRequest(request_id=str(i), input_ids=[0] * int(rng.integers(20, 700)),
                                       max_new_tokens=int(rng.integers(2, 6))))
    checked = 0
    for _ in range(12):
        plan = s.plan_step()
        if plan is None:
            break
        T, nd, n = plan.num_tokens, plan.num_decode, plan.num_entries
        k = torch.randn(T, 1, 256, device=DEV, generator=g).bfloat16()
        v = torch.randn(T, 1, 256, device=DEV, generator=g).bfloat16()
        cache.append(plan.slot_mapping, k, v, layer=0)
        if n > nd:
            cu = plan.cu_seqlens[nd:] - plan.cu_seqlens[nd]
            t0 = int(plan.cu_seqlens[nd].item())
            q = torch.randn(T - t0, 4, 256, device=DEV, generator=g).bfloat16()
            width = plan.block_tables.shape[1]
            out = A.attn_prefill_paged(q, *cache.get_kv_by_layer(0), cu, plan.seq_lens[nd:],
                                       plan.block_tables[nd:], max(c for _, _, c in plan.prefill))
            torch.cuda.synchronize()
            A.check_errors(DEV)
            kc, vc = cache.get_kv_by_layer(0)
            want = att.prefill_attention(q.float().cpu().numpy(), kc.float().cpu().numpy(),
                                         vc.float().cpu().numpy(), cu.cpu().numpy(), 256 ** -0.5,
                                         True, lens_k=plan.seq_lens[nd:].cpu().numpy(),
                                         page_table=plan.block_tables[nd:].cpu().numpy(),
                                         stats=True)
            within(out, want)
            assert width >= 1
            checked += 1
        s.complete_step(plan)
    s.check_errors()
    assert checked >= 3


def test_bad_page_and_bad_offsets_are_flagged():
    case("attn_prefill_paged bad page id; attn_prefill offsets past the buffer")
    g = torch.Generator().manual_seed(37)
    kc = torch.randn(8, 16, 1, 256, generator=g).bfloat16().to(DEV)
    vc = torch.randn(8, 16, 1, 256, generator=g).bfloat16().to(DEV)
    q = torch.randn(20, 4, 256, generator=g).bfloat16().to(DEV)
    table = torch.tensor([[1, 99]], dtype=torch.int32, device=DEV)
    cu = torch.tensor([0, 20], dtype=torch.int32, device=DEV)
    A.attn_prefill_paged(q, kc, vc, cu, torch.tensor([30], dtype=torch.int32, device=DEV), table,
                         20)
    with pytest.raises(_lib.MkvDeviceError, match="page id"):
        A.check_errors(DEV)
    k = torch.randn(20, 1, 256, generator=g).bfloat16().to(DEV)
    cu_k = torch.tensor([0, 25], dtype=torch.int32, device=DEV)  # past the 20 key rows
    A.attn_prefill(q, k, k.clone(), cu, cu_k, 20, 25)
    with pytest.raises(_lib.MkvDeviceError, match="table"):
        A.check_errors(DEV)


@pytest.mark.parametrize("split_len", [64, 128, 192])
def test_forced_key_splits_through_the_c_abi(split_len):
    """Key ranges of one, two and three 64-key tiles (the double-buffered
    loop's prologue-only, one-store and store-plus-prefetch cases), ranges
    that end inside a sequence or past its causal limit, and the merge, with
    the split chosen by the caller of the C ABI."""
    lens = [1, 63, 64, 65, 128, 129, 200, 383]
    case(f"mkv_prefill_attention_bf16 forced split_len {split_len}, lens {lens}")
    _forced_splits(lens, split_len, 38 + split_len)


@pytest.mark.parametrize("splits", [2, 3, 4, 5, 6, 7, 8, 9])
def test_every_merged_range_count(splits):
    """64-key ranges, as many as `splits`: the merge reads each count from 2
    to 8 with its own fixed number of loads and more than 8 through a loop;
    sequences end inside, at and past the ranges' edges."""
    lens = [1, 63, 64, 65, 64 * splits - 1, 64 * splits]
    case(f"mkv_prefill_attention_bf16 {splits} ranges of 64 keys, lens {lens}")
    _forced_splits(lens, 64, 60 + splits)


def _forced_splits(lens, split_len, seed):
    g, cu = seqs(lens, seed)
    T, max_k = int(cu[-1]), max(lens)
    q = torch.randn(T, 4, 256, generator=g).bfloat16().to(DEV)
    k = torch.randn(T, 1, 256, generator=g).bfloat16().to(DEV)
    v = torch.randn(T, 1, 256, generator=g).bfloat16().to(DEV)
    splits = -(-max_k // split_len)
    lib = _lib.load()
    ws_bytes = lib.mkv_prefill_attention_workspace_bytes(T, 4, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    cu_d = cu.to(DEV)
    _lib.call("mkv_prefill_attention_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), T, 1, 4, 256,
              None, 0, 0, cu_d.data_ptr(), cu_d.data_ptr(), None, len(lens), T, max_k,
              256 ** -0.5, 1, splits, split_len, out.data_ptr(), ws.data_ptr(), ws_bytes,
              A._errword(DEV).ptr(), _lib.stream_of(DEV))
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = att.prefill_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                 v.float().cpu().numpy(), cu.numpy(), 256 ** -0.5, True,
                                 cu_k=cu.numpy(), stats=True)
    within(out, want)


def _one_hot_keys(n_rows, heads=1):
    """V row j = e_(j mod 256) (bf16 ones): with a zero query every visible
    key has weight 1 / n, so output dim d is (visible keys j = d mod 256) / n
    and one key more or less changes a dim by about 1 / n, far above the
    rounding (the worst-case tolerance above cannot see a single key once a
    row attends to a few hundred)."""
    v = torch.zeros(n_rows, heads, 256)
    idx = torch.arange(n_rows)
    v[idx, :, idx % 256] = 1.0
    return v.bfloat16()


def _one_hot_want(nq, nk, causal):
    """Closed form for a zero query over one-hot keys: [nq, 256] float64."""
    out = np.zeros((nq, 256))
    d = np.arange(256)
    for t in range(nq):
        last = nk - nq + t if causal else nk - 1  # bottom-right causal alignment
        if last < 0:
            continue
        n = last + 1
        cnt = np.where(d <= last, (last - d) // 256 + 1, 0)
        out[t] = cnt / n
    return out


def _bf16_close(got, want):
    got = got.float().cpu().numpy().astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    err = np.abs(got - want)
    assert (err <= ulp).all(), f"worst {err.max()} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("causal", [True, False])
def test_understated_max_seqlen_k_keeps_every_key(causal):
    """A max_seqlen_k below the real key count (600 for 2000 keys): the split
    ranges cover 3 x 256 keys, and the last range must run to the end."""
    nq = nk = 2000
    case(f"attn_prefill one-hot keys, {nk} keys, max_seqlen_k 600, causal={causal}")
    q = torch.zeros(nq, 4, 256).bfloat16().to(DEV)
    k = torch.randn(nk, 1, 256, generator=torch.Generator().manual_seed(41)).bfloat16().to(DEV)
    v = _one_hot_keys(nk).to(DEV)
    cu = torch.tensor([0, nq], dtype=torch.int32, device=DEV)
    out = A.attn_prefill(q, k, v, cu, cu, nq, 600, causal=causal)
    torch.cuda.synchronize()
    A.check_errors(DEV)
    want = _one_hot_want(nq, nk, causal)
    for h in range(4):
        _bf16_close(out[:, h], want)


def test_one_hot_keys_pin_every_tile_and_split_boundary():
    """Sequences with a prefix (nk > nq) and lengths around the 64-key tiles
    and the split boundaries, with forced key splits through the C ABI: each
    output dim counts its visible keys exactly, so a key dropped or added at
    any tile or range boundary shows."""
    nqs = [1, 63, 64, 65, 129, 300]
    nks = [1, 64, 127, 65, 300, 777]
    case(f"mkv_prefill_attention_bf16 one-hot keys, forced splits of 128, nq {nqs} nk {nks}")
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(nqs)]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(nks)]), dtype=torch.int32)
    Tq, Tk = int(cu_q[-1]), int(cu_k[-1])
    q = torch.zeros(Tq + 7, 4, 256).bfloat16().to(DEV)  # 7 rows past every sequence
    k = torch.randn(Tk, 1, 256, generator=torch.Generator().manual_seed(42)).bfloat16().to(DEV)
    v = torch.cat([_one_hot_keys(n) for n in nks]).to(DEV)
    split_len, max_k = 128, max(nks)
    splits = -(-max_k // split_len)
    lib = _lib.load()
    ws_bytes = lib.mkv_prefill_attention_workspace_bytes(Tq + 7, 4, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    canary = torch.full((Tq + 7, 4, 256), 0x1234, dtype=torch.int16, device=DEV)
    out = canary.clone().view(torch.bfloat16)
    cu_qd, cu_kd = cu_q.to(DEV), cu_k.to(DEV)
    _lib.call("mkv_prefill_attention_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), Tk, 1, 4,
              256, None, 0, 0, cu_qd.data_ptr(), cu_kd.data_ptr(), None, len(nqs), Tq + 7,
              max(nqs), 256 ** -0.5, 1, splits, split_len, out.data_ptr(), ws.data_ptr(),
              ws_bytes, A._errword(DEV).ptr(), _lib.stream_of(DEV))
    torch.cuda.synchronize()
    A.check_errors(DEV)
    for b, (nq, nk) in enumerate(zip(nqs, nks)):
        want = _one_hot_want(nq, nk, True)
        rows = out[int(cu_q[b]):int(cu_q[b + 1])]
        for h in range(4):
            _bf16_close(rows[:, h], want)
    # rows outside every sequence's queries are left alone by the merge
    assert torch.equal(out[Tq:].view(torch.int16), canary[Tq:])
