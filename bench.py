"""Benchmark of the KV-cache hot path on one MI355X.

Default workload (the headline metric): decode-step append + padded gather on
one tensor-parallel rank — 15 attention layers, 1 KV head of 256, bf16 pool,
16-token pages, batch 256, context lengths log-normal (median 4096, sigma 1,
clipped to [1, 32768], seed 102). One step = one new token per sequence per
layer appended through the slot mapping, and per layer a gather of every
block table into padded contiguous [256, Lpad, 1, 256] K and V (zero padding).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Prints one JSON line. ``value`` is algorithmic HBM bytes per step / step
time (GB/s); ``roofline`` is the gather kernel's algorithmic bytes per launch
/ its mean launch time from HIP events on its stream, against 8 TB/s;
``cpu_baseline`` times the CPU oracle (torch-CPU restatement of the reference)
on 3 whole decode steps (15 layers of append + padded gather) on the host's
cores, after which the GPU runs the same 3 steps and the pools are compared.
After the headline's timed region, the default run also measures the other
configurations (``secondary``): fp8 chunked prefill (append and dequant-gather
separately), the GDN state slots in model order and MALL-cold, the prefix
cache (us per request, hashing and block manager apart), and paged decode
attention over bf16 and fp8 pools at the headline's shape (200 steps).
"""
from __future__ import annotations

import argparse
import ctypes
import gc
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of 8 TB/s) for KV append+gather; decode step µs @ batch 256"

B = 256
LAYERS = 15
HEAD_DIM = 256
ROW = HEAD_DIM * 2  # bytes per token row (1 head, bf16)
SEED = 102
PLACEMENT = "shuffled"  # fp8_prefill page placement (--placement)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def context_lengths(seed: int = SEED) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.clip(np.round(rng.lognormal(np.log(4096.0), 1.0, B)), 1, 32768).astype(np.int64)


def prefix_requests(n_requests: int, seed: int = 104, n_templates: int = 64,
                    template_len: int = 4096, suffix: tuple[int, int] = (64, 1024),
                    zipf_s: float = 1.1, vocab: int = 151936) -> list[np.ndarray]:
    """Prompts = one of n_templates seeded templates of template_len random
    token ids in [0, vocab), drawn by a bounded Zipf(s) law over the templates,
    plus a random suffix of suffix[0]..suffix[1] ids (int64)."""
    rng = np.random.default_rng(seed)
    templates = rng.integers(0, vocab, (n_templates, template_len), dtype=np.int64)
    p = np.arange(1, n_templates + 1, dtype=np.float64) ** -zipf_s
    choice = rng.choice(n_templates, size=n_requests, p=p / p.sum())
    lens = rng.integers(suffix[0], suffix[1] + 1, n_requests)
    return [np.concatenate([templates[c], rng.integers(0, vocab, int(n), dtype=np.int64)])
            for c, n in zip(choice, lens)]


def prefix_ops(n_requests: int, batch: int) -> list[list[int]]:
    """Per batch: release the previous batch's requests, then admit this one's."""
    out = []
    for b0 in range(0, n_requests, batch):
        prev = range(max(0, b0 - batch), b0)
        out.append([-(r + 1) for r in prev] + list(range(b0, min(n_requests, b0 + batch))))
    return out


def step_bytes(lens: np.ndarray) -> tuple[float, float, float]:
    """(all algorithmic bytes of one step, of one gather launch, useful bytes of
    one step without padding writes) for post-append lengths ``lens``."""
    lpad = int(-(-int(lens.max()) // 16) * 16)
    nblk = -(-lens // 16)
    gather = 2 * ROW * lens.sum() + 2 * ROW * B * lpad + 4 * nblk.sum() + 4 * B
    append = 2 * B * ROW + 2 * B * ROW + 8 * B
    useful = 2 * B * ROW + 2 * B * ROW + 8 * B + 4 * ROW * lens.sum() + 4 * nblk.sum() + 4 * B
    return float(LAYERS * (gather + append)), float(gather), float(LAYERS * useful)


CPU_STEPS = 3  # whole decode steps the CPU baseline times


def cpu_threads() -> dict:
    """Sets torch's CPU threads to every core this process may run on (its
    affinity set, capped by OMP_NUM_THREADS where the host sets it: a shared
    host gives one GPU's job a share of its cores) and describes them."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(affinity, int(omp)) if omp.isdigit() and int(omp) > 0 else affinity
    torch.set_num_threads(threads)
    return {"cores": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
            "affinity_cpus": affinity, "omp_num_threads": omp or None, "cpu_model": _cpu_model()}


def cpu_baseline_steps(cache, seqs, kin, vin, first: int, n_steps: int, gpu_step) -> dict:
    """The oracle's decode step on the host's cores, for n_steps whole steps
    (the slot assignment of oracle.paged.decode_step, then per layer the
    slot-mapped append and the padded gather of K and V: torch-CPU
    index_put_ / index_select, restating muserve/kv_cache.py:102-158 and the
    [B,S,H,D] layout of muserve/model/qwen35_model.py:223-249), on a copy of
    the device KV pool taken after the timed loop, with the inputs of steps
    first .. first+n_steps-1. The GPU then runs the same steps (gpu_step) and
    its pool and last gather are compared with the CPU's byte for byte."""
    from oracle import paged as ref

    info = cpu_threads()
    cpu_cache = cache.cache.cpu()
    pool = ref.PoolModel(cache.num_pages, list(cache._free_pages))
    oseqs = []
    for s in seqs:
        o = ref.SeqModel()
        o.page_table, o.seq_len = list(s.page_table), s.seq_len
        oseqs.append(o)
    k_cpu = kin[first:first + n_steps].cpu()
    v_cpu = vin[first:first + n_steps].cpu()
    nbytes = 0.0
    t0 = time.perf_counter()
    for j in range(n_steps):
        slots = torch.tensor(ref.decode_step(pool, oseqs), dtype=torch.int64)
        lens = np.array([o.seq_len for o in oseqs], dtype=np.int64)
        width = max(len(o.page_table) for o in oseqs)
        table = np.zeros((len(oseqs), width), dtype=np.int32)
        for b, o in enumerate(oseqs):
            table[b, :len(o.page_table)] = o.page_table
        bt = torch.from_numpy(table)
        sl = torch.from_numpy(lens.astype(np.int32))
        lpad = int(-(-int(lens.max()) // 16) * 16)
        for l in range(LAYERS):
            ref.append(cpu_cache, slots, k_cpu[j, l], v_cpu[j, l], layer=l)
            k_ref = ref.gather_padded(cpu_cache[l, 0], bt, sl, lpad)
            v_ref = ref.gather_padded(cpu_cache[l, 1], bt, sl, lpad)
        nbytes += step_bytes(lens)[0]
    dt = time.perf_counter() - t0
    for j in range(n_steps):
        kout, vout = gpu_step(first + j)
    torch.cuda.synchronize()
    cache.check_errors()
    same_gather = bool(torch.equal(kout.cpu().view(torch.int16), k_ref.view(torch.int16)) and
                       torch.equal(vout.cpu().view(torch.int16), v_ref.view(torch.int16)))
    same_pool = all(torch.equal(cache.cache[l].cpu().view(torch.int16),
                                cpu_cache[l].view(torch.int16)) for l in range(LAYERS))
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        **info,
        "kind": "port",
        "sample": (f"{n_steps} whole decode steps of the oracle (slot assignment, then per layer "
                   f"the append and the padded K/V gather, torch-CPU, {info['cores']} threads) at "
                   f"batch {B}, {LAYERS} layers, Lpad {lpad}: {dt:.2f} s, "
                   f"{1e3 * dt / n_steps:.0f} ms per step"),
        "seconds": round(dt, 3),
        "ms_per_step": round(1e3 * dt / n_steps, 1),
        "gpu_pool_matches_cpu_after_the_steps": same_pool,
        "gpu_last_gather_matches_cpu": same_gather,
    }


PMC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "gather_decode_b256_hbm_counters.md")


def counter_traffic() -> tuple[float | None, float | None]:
    """(HBM bytes per gather launch, traffic/algorithmic ratio) recorded from
    the FETCH_SIZE/WRITE_SIZE runs of this workload, if that summary exists."""
    vals = {}
    try:
        for line in open(PMC_PROFILE):
            if ":" in line and line.split(":", 1)[0].strip() in (
                    "traffic_bytes_per_gather_launch", "traffic_to_algorithmic_ratio"):
                k, v = line.split(":", 1)
                vals[k.strip()] = float(v)
    except OSError:
        pass
    return vals.get("traffic_bytes_per_gather_launch"), vals.get("traffic_to_algorithmic_ratio")


def counter_ratios(name: str) -> dict[str, float]:
    """Per-kernel HBM traffic / algorithmic-byte ratios ("ratio <kernel>: x"
    lines) recorded in profiles/<name> from its FETCH_SIZE/WRITE_SIZE runs."""
    out = {}
    try:
        for line in open(os.path.join(os.path.dirname(PMC_PROFILE), name)):
            if line.startswith("ratio ") and ":" in line:
                k, v = line[len("ratio "):].split(":", 1)
                out[k.strip()] = float(v)
    except OSError:
        pass
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_decode(steps: int, warmup: int, with_cpu: bool) -> dict:
    from muserve_amd.kv_cache import BlockTables, PagedKVCache, SequenceKVState, reserve_tokens

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = context_lengths()
    # the CPU baseline's steps run on the GPU too, after the timed loop
    total_steps = warmup + steps + (CPU_STEPS if with_cpu else 0)
    pages = int(np.sum(-(-(ctx + total_steps) // 16))) + 64
    log(f"pool: {pages} pages x {LAYERS} layers (ctx sum {int(ctx.sum())}, max {int(ctx.max())})")
    cache = PagedKVCache(pages, num_layers=LAYERS, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=torch.bfloat16, device=dev, verbose=False)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    for l in range(LAYERS):  # pool contents ~N(0,1)
        cache.cache[l].normal_(generator=gen)
    cache.shuffle_free_list(torch.Generator().manual_seed(SEED))
    seqs = [SequenceKVState() for _ in range(B)]
    for s, n in zip(seqs, ctx):
        reserve_tokens(cache, s, int(n))
    width = int(-(-(int(ctx.max()) + total_steps) // 16))
    bt = BlockTables(cache, seqs, max_pages=width)
    # per-step new K/V, ~N(0,1), resident before timing: [steps, L, B, 1, 256]
    kin = torch.empty(total_steps, LAYERS, B, 1, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vin = torch.empty_like(kin)
    kin.normal_(generator=gen)
    vin.normal_(generator=gen)
    lpad_max = int(-(-(int(ctx.max()) + total_steps) // 16) * 16)
    kbuf = torch.empty(B * lpad_max * HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vbuf = torch.empty_like(kbuf)
    stream = torch.cuda.current_stream(dev)
    stamps = Stamps()

    def one_step(i: int, rec=None, steps_rec=None):
        step = stamps.span(stream) if steps_rec is not None else None
        slots = bt.decode_step()
        lpad = bt.padded_len()
        kout = kbuf[:B * lpad * HEAD_DIM].view(B, lpad, 1, HEAD_DIM)
        vout = vbuf[:B * lpad * HEAD_DIM].view(B, lpad, 1, HEAD_DIM)
        for l in range(LAYERS):
            cache.append(slots, kin[i, l], vin[i, l], layer=l)
            sp = stamps.span(stream) if rec is not None else None
            cache.gather(l, bt.tables, bt.seq_lens, out_len=lpad, out=(kout, vout))
            if rec is not None:
                rec.append(("gather", sp.end(stream)))
        if steps_rec is not None:
            steps_rec.append(step.end(stream))
        return kout, vout

    log(f"warmup {warmup} steps")
    for i in range(warmup):
        one_step(i)
    torch.cuda.synchronize()
    cache.check_errors()

    lens0 = bt._lens.copy()
    all_bytes = gather_bytes = useful = 0.0
    for j in range(steps):  # lengths after step j's append are lens0 + j + 1
        a, g_, u = step_bytes(lens0 + j + 1)
        all_bytes += a
        gather_bytes += g_
        useful += u
    recs = [[] for _ in range(steps)]
    step_spans: list = []
    log(f"timing {steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for j in range(steps):
        one_step(warmup + j, recs[j], step_spans)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    cache.check_errors()
    mean_gather_s = _timed(recs, "gather") / 1e3
    mean_gather_bytes = gather_bytes / steps

    traffic, ratio = counter_traffic()
    step_s = elapsed / steps
    value = all_bytes / elapsed / 1e9
    achieved = mean_gather_bytes / mean_gather_s / 1e9
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded ~N(0,1) K/V, seeded log-normal context lengths)",
        "config": {
            "workload": ("decode-step KV append + padded block-table gather on one TP rank: "
                         "15 attention layers, batch 256, 1 KV head x 256, bf16, 16-token pages, "
                         "ctx lognormal(median 4096, sigma 1.0, clip 1..32768), seed 102"),
            "batch": B, "layers": LAYERS, "kv_heads": 1, "head_dim": HEAD_DIM, "page_size": 16,
            "ctx_sum_start": int(lens0.sum()), "ctx_max_start": int(lens0.max()),
        },
        "decode_step_us": round(step_s * 1e6, 1),
        "step_time": _step_stats(step_spans),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(B / step_s, 1),
        "useful_GBps_without_padding_writes": round(useful / elapsed / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "mkv_gather_bf16 = gather_pad_kernel<512> + gather_data_kernel<512>",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            # HBM bytes per launch: the FETCH_SIZE/WRITE_SIZE runs' traffic-to-
            # algorithmic ratio applied to this run's mean launch (the profiled
            # launches had the same workload at its first steps' lengths)
            "traffic": round(ratio * mean_gather_bytes) if ratio else None,
            "traffic_to_algorithmic": ratio,
            "traffic_profiled_bytes_per_launch": traffic,
            "traffic_source": ("rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 (scales from a 1 GiB copy), "
                               "profiles/gather_decode_b256_hbm_counters.md"),
            "mean_launch_us": round(mean_gather_s * 1e6, 2),
            "algorithmic_bytes_per_launch": round(mean_gather_bytes),
        },
    }
    if with_cpu:
        log(f"cpu baseline ({CPU_STEPS} whole steps of the oracle)")
        res["cpu_baseline"] = cpu_baseline_steps(cache, seqs, kin, vin, warmup + steps, CPU_STEPS,
                                                 one_step)
    return res


class Stamps:
    """Timing events of the timed regions: HIP events created with
    hipEventDisableSystemFence, recorded on torch's streams. A default event's
    system-scope release (an L2 write-back) adds ~3 us to every launch it
    brackets on MI355X; these agree with rocprof's kernel times within ~1 us.
    Read after a synchronize."""
    _NO_SYSTEM_FENCE = 0x20000000

    def __init__(self):
        from muserve_amd import _lib
        paths = _lib._hip_runtimes()
        if len(paths) != 1:
            raise RuntimeError(f"expected exactly one HIP runtime mapped, found {paths}")
        hip = ctypes.CDLL(paths[0])
        hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                            ctypes.c_void_p]
        hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        hip.hipStreamWaitEvent.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint]
        self._hip = hip
        self._events: list[ctypes.c_void_p] = []

    def record(self, stream) -> ctypes.c_void_p:
        ev = ctypes.c_void_p()
        if self._hip.hipEventCreateWithFlags(ctypes.byref(ev), self._NO_SYSTEM_FENCE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")
        if self._hip.hipEventRecord(ev, ctypes.c_void_p(stream.cuda_stream)) != 0:
            raise RuntimeError("hipEventRecord failed")
        self._events.append(ev)
        return ev

    def wait(self, stream, ev: ctypes.c_void_p) -> None:
        """Work queued on ``stream`` after this waits for ``ev``."""
        if self._hip.hipStreamWaitEvent(ctypes.c_void_p(stream.cuda_stream), ev, 0) != 0:
            raise RuntimeError("hipStreamWaitEvent failed")

    def ms(self, a: ctypes.c_void_p, b: ctypes.c_void_p) -> float:
        out = ctypes.c_float()
        if self._hip.hipEventElapsedTime(ctypes.byref(out), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return float(out.value)

    def span(self, stream) -> "Span":
        return Span(self, stream)

    def close(self) -> None:
        for ev in self._events:
            self._hip.hipEventDestroy(ev)
        self._events.clear()


class Span:
    """A start event recorded now; end() records the stop event."""

    def __init__(self, stamps: Stamps, stream):
        self._s = stamps
        self._a = stamps.record(stream)
        self._b = None

    def end(self, stream) -> "Span":
        self._b = self._s.record(stream)
        return self

    def ms(self) -> float:
        return self._s.ms(self._a, self._b)


def _timed(recs: list, label: str) -> float:
    """Mean milliseconds of the spans recorded under label (recs: per step,
    lists of (label, Span))."""
    ms = [sp.ms() for step in recs for (lab, sp) in step if lab == label]
    return float(np.mean(ms)) if ms else float("nan")


def _step_stats(spans: list) -> dict:
    """Median / p10 / p90 of per-step times (ms)."""
    ms = np.array([sp.ms() for sp in spans])
    return {"median_ms": round(float(np.median(ms)), 4),
            "p10_ms": round(float(np.percentile(ms, 10)), 4),
            "p90_ms": round(float(np.percentile(ms, 90)), 4)}


def _kernel_roofline(name: str, nbytes: float, ms: float, ratio: float | None = None) -> dict:
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"kernel": name, "bound": "hbm", "algorithmic_bytes_per_launch": round(nbytes),
            "mean_launch_us": round(ms * 1e3, 2), "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": round(ratio * nbytes) if ratio else None, "traffic_to_algorithmic": ratio}


def _roofline_of(kernels: list[dict], profile: str) -> dict:
    """The contract's roofline object for the kernel with the most time per
    step (first in ``kernels`` by convention), plus every kernel's entry."""
    top = dict(kernels[0])
    top["traffic_source"] = (f"rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 (scales from a 1 GiB "
                             f"copy), profiles/{profile}")
    top["kernels"] = kernels
    return top


def run_fp8_prefill(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Chunked prefill into an fp8 pool: 32 requests append 2048-token chunks
    (bf16 ~N(0,1), 1 % of elements x20) into 128k-token contexts, quantised on
    append (per-token absmax/448 scale), then a dequant-gather of the last 8192
    tokens of every request; 15 layers, 1 KV head x 256."""
    from muserve_amd.kv_cache import PagedKVCache, SequenceKVState, reserve_tokens, slot_mapping_for

    R, CHUNK, CTX, WIN, L = 32, 2048, 131072, 8192, LAYERS
    n_chunks = warmup + steps
    if CHUNK * n_chunks > CTX - WIN:
        raise SystemExit(f"at most {(CTX - WIN) // CHUNK} chunks fit in a {CTX}-token context")
    prior = CTX - CHUNK * n_chunks
    dev = torch.device("cuda:0")
    pages = R * CTX // 16 + 16
    cache = PagedKVCache(pages, num_layers=L, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=torch.float8_e4m3fn, device=dev, verbose=False)
    if PLACEMENT == "shuffled":
        cache.shuffle_free_list(torch.Generator().manual_seed(103))
    # "contiguous": the LIFO free list hands each request consecutive pages
    gen = torch.Generator(device=dev).manual_seed(103)

    def kv_batch(t: int) -> torch.Tensor:
        x = torch.randn(L, t, 1, HEAD_DIM, generator=gen, device=dev)
        boost = torch.rand(L, t, 1, HEAD_DIM, generator=gen, device=dev) < 0.01
        return torch.where(boost, x * 20.0, x).bfloat16()

    seqs = [SequenceKVState() for _ in range(R)]
    log(f"fp8 pool {pages} pages; prefilling {prior} tokens x {R} requests")
    step = 8192
    for s0 in range(0, prior, step):
        n = min(step, prior - s0)
        slots = np.concatenate([slot_mapping_for(sq, reserve_tokens(cache, sq, n), n) for sq in seqs])
        sl = torch.from_numpy(slots).to(dev)
        cache.append(sl, kv_batch(len(slots)), kv_batch(len(slots)))
    # the chunks' pages and slot mappings, resident before timing
    slot_steps, lens_steps = [], []
    for _ in range(n_chunks):
        slot_steps.append(np.concatenate(
            [slot_mapping_for(sq, reserve_tokens(cache, sq, CHUNK), CHUNK) for sq in seqs]))
        lens_steps.append([sq.seq_len for sq in seqs])
    width = CTX // 16
    bt = torch.zeros(R, width, dtype=torch.int32)
    for b, sq in enumerate(seqs):
        bt[b, :len(sq.page_table)] = torch.tensor(sq.page_table, dtype=torch.int32)
    bt = bt.to(dev)
    slots_dev = torch.from_numpy(np.stack(slot_steps)).to(dev)
    lens_dev = torch.tensor(lens_steps, dtype=torch.int32, device=dev)
    starts_dev = (lens_dev - WIN).clamp(min=0).contiguous()
    # every request holds more than WIN tokens, so the windows are full and the
    # packed layout at row offsets b*WIN is the padded [R, WIN, 1, 256] output
    assert min(min(x) for x in lens_steps) >= WIN
    cu_out = torch.arange(R + 1, dtype=torch.int64, device=dev) * WIN
    T = R * CHUNK
    kin = torch.stack([kv_batch(T) for _ in range(n_chunks)])
    vin = torch.stack([kv_batch(T) for _ in range(n_chunks)])
    kbuf = torch.empty(R, WIN, 1, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vbuf = torch.empty_like(kbuf)
    torch.cuda.synchronize()
    cache.check_errors()
    stream = torch.cuda.current_stream(dev)
    stamps = Stamps()

    # A step appends the chunk's K/V of all 15 layers in one launch (the
    # chunk's [L, T, 1, 256] inputs are all there when the step starts), then
    # dequant-gathers every layer's window. One event pair brackets the append
    # and one each group of 15 gathers, so the mean launch time carries no
    # per-launch event overhead. The per-layer form (15 launches, as a layer
    # loop issues them) is timed after the timed region.
    def one_step(i: int, rec=None, steps_rec=None):
        step = stamps.span(stream) if steps_rec is not None else None
        sp = stamps.span(stream) if rec is not None else None
        cache.append(slots_dev[i], kin[i], vin[i])
        if rec is not None:
            rec.append(("append", sp.end(stream)))
            sp = stamps.span(stream)
        for l in range(L):
            cache.gather(l, bt, lens_dev[i], out_len=WIN, starts=starts_dev[i], out=(kbuf, vbuf),
                         cu_out=cu_out)
        if rec is not None:
            rec.append(("gather", sp.end(stream)))
        if steps_rec is not None:
            steps_rec.append(step.end(stream))

    for i in range(warmup):
        one_step(i)
    torch.cuda.synchronize()
    recs = [[] for _ in range(steps)]
    step_spans: list = []
    t0 = time.perf_counter()
    for j in range(steps):
        one_step(warmup + j, recs[j], step_spans)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    cache.check_errors()
    # The per-layer form, over the timed steps' chunks again: the same bytes
    # into the same slots, so the pool ends as it was.
    per_layer = [[] for _ in range(steps)]
    for j in range(steps):
        i = warmup + j
        sp = stamps.span(stream)
        for l in range(L):
            cache.append(slots_dev[i], kin[i, l], vin[i, l], layer=l)
        per_layer[j].append(("append", sp.end(stream)))
    torch.cuda.synchronize()
    cache.check_errors()
    ratios = counter_ratios("fp8_prefill_hbm_counters.md")
    append_bytes = T * (1024 + 512 + 8 + 8)
    gather_bytes = R * WIN * (520 + 1024) + R * (WIN // 16 + 1) * 4 + 8 * R
    step_bytes_ = L * (append_bytes + gather_bytes)
    step_s = elapsed / steps
    res = {
        "metric": "achieved HBM GB/s (% of 8 TB/s) for fp8 quantize-on-append + dequant-gather",
        "value": round(step_bytes_ / step_s / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3fn",
        "data": "synthetic (seeded ~N(0,1) bf16 K/V with 1% x20 outliers)",
        "config": {"workload": ("fp8 chunked prefill: 32 requests x 2048-token chunks into 128k "
                                "contexts, 15 layers, 1 KV head x 256, e4m3fn + fp32 per-token "
                                "scale, then dequant-gather of the last 8192 tokens; seed 103"),
                   "page_placement": PLACEMENT},
        "appended_tokens_per_s": round(T / step_s, 1),
        "step_time": _step_stats(step_spans),
        "pct_of_hbm_peak": round(100 * step_bytes_ / step_s / 1e9 / HBM_PEAK_GBS, 2),
        "roofline": _roofline_of([
            _kernel_roofline("gather_dequant_kernel<1> (mkv_gather_dequant_fp8)", gather_bytes,
                             _timed(recs, "gather") / L, ratios.get("gather_dequant_kernel")),
            _kernel_roofline("append_fp8_kernel<1> (mkv_append_fp8, 15 layers in one launch)",
                             L * append_bytes, _timed(recs, "append"),
                             ratios.get("append_fp8_kernel")),
            _kernel_roofline("append_fp8_kernel<1> (mkv_append_fp8, one launch per layer)",
                             append_bytes, _timed(per_layer, "append") / L,
                             ratios.get("append_fp8_kernel_per_layer"))],
            "fp8_prefill_hbm_counters.md"),
    }
    if with_cpu:
        from oracle import fp8 as ref
        n = 2048
        x = kin[warmup + steps - 1, 0, :n].cpu()
        t1 = time.perf_counter()
        q, sc = ref.quantize_rows(x)
        dt = time.perf_counter() - t1
        pg = slots_dev[warmup + steps - 1, :n].cpu()
        got_q = cache.cache[0, 0].view(torch.uint8).reshape(-1, 1, HEAD_DIM)[pg].cpu()
        got_s = cache.scales[0, 0].reshape(-1, 1)[pg].cpu()
        res["cpu_baseline"] = {
            "value": round(n * (1024 + 512 + 8) / 2 / dt / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle quantize_rows (torch-CPU) of {n} K rows of one layer: {dt*1e3:.1f} ms",
            "gpu_matches_cpu_on_sample": bool(torch.equal(got_q, q) and torch.equal(
                got_s.view(torch.int32), sc.view(torch.int32)))}
    return res


def run_gdn_state(steps: int, warmup: int, with_cpu: bool, fused_conv: bool = False) -> dict:
    """Decode step of the hybrid stack, 60 layers in model order: each GDN
    layer gathers the 256 active requests' recurrent [8,128,128] fp32 + conv
    [2048,4] bf16 states from a 1024-slot pool (seeded permuted slots),
    updates them (a synthetic +1, timed apart) and scatters them back; each
    attention layer (l % 4 == 3) appends one decode token per request (the
    headline workload's appends). fused_conv: the conv states are not
    gathered; each GDN layer runs the decode conv in place on them
    (StatePool.conv_decode: one token's mixed_qkv per request in, silu(conv)
    out, state shifted), and only the recurrent states are gathered, updated
    and scattered."""
    from muserve_amd.kv_cache import BlockTables, PagedKVCache, SequenceKVState, reserve_tokens
    from muserve_amd.state_pool import StatePool, gdn_ordinal

    dev = torch.device("cuda:0")
    S, G = 1024, 45
    pool = StatePool(num_layers=G, num_slots=S, device=dev)
    gen = torch.Generator(device=dev).manual_seed(105)
    pool.state.normal_(generator=gen)
    pool.conv.normal_(generator=gen)
    slots = torch.randperm(S, generator=torch.Generator().manual_seed(105))[:B].to(
        torch.int32).to(dev)
    ctx = context_lengths()
    total = warmup + steps
    pages = int(np.sum(-(-(ctx + total) // 16))) + 64
    cache = PagedKVCache(pages, num_layers=LAYERS, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=torch.bfloat16, device=dev, verbose=False)
    cache.shuffle_free_list(torch.Generator().manual_seed(SEED))
    seqs = [SequenceKVState() for _ in range(B)]
    for s_, n in zip(seqs, ctx):
        reserve_tokens(cache, s_, int(n))
    bt = BlockTables(cache, seqs, max_pages=int(-(-(int(ctx.max()) + total) // 16)))
    kin = torch.randn(total, LAYERS, B, 1, HEAD_DIM, generator=gen, device=dev).bfloat16()
    vin = torch.randn(total, LAYERS, B, 1, HEAD_DIM, generator=gen, device=dev).bfloat16()
    # the layer's working set: the batch's states, contiguous
    sbuf = torch.empty((B, *pool.state.shape[2:]), dtype=pool.state.dtype, device=dev)
    cbuf = torch.empty((B, *pool.conv.shape[2:]), dtype=pool.conv.dtype, device=dev)
    C = pool.conv.shape[2]
    if fused_conv:  # a ring of 4 steps of per-request conv inputs, the layers' weights
        xin = torch.randn(4, G, B, C, generator=gen, device=dev).bfloat16()
        wconv = (0.5 * torch.randn(G, C, 1, 4, generator=gen, device=dev)).bfloat16()
        cout = torch.empty(B, C, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    stamps = Stamps()

    def one_step(i: int, rec=None, steps_rec=None):
        step = stamps.span(stream) if steps_rec is not None else None
        kv_slots = bt.decode_step()
        for layer in range(60):
            if layer % 4 == 3:
                a = layer // 4
                cache.append(kv_slots, kin[i, a], vin[i, a], layer=a)
                continue
            g = gdn_ordinal(layer)
            sp = stamps.span(stream) if rec is not None else None
            if fused_conv:  # recurrent gather + conv in place, one launch
                pool.decode_gather(g, slots, xin[i % 4, g], wconv[g], state_out=sbuf,
                                   conv_out=cout)
            else:
                pool.gather(g, slots, out=(sbuf, cbuf))
            if rec is not None:
                rec.append(("gather", sp.end(stream)))
                sp = stamps.span(stream)
            sbuf.add_(1.0)
            if not fused_conv:
                cbuf.add_(1.0)
            if rec is not None:
                rec.append(("update", sp.end(stream)))
                sp = stamps.span(stream)
            pool.scatter(g, slots, sbuf, None if fused_conv else cbuf)
            if rec is not None:
                rec.append(("scatter", sp.end(stream)))
        if steps_rec is not None:
            steps_rec.append(step.end(stream))

    for i in range(warmup):
        one_step(i)
    torch.cuda.synchronize()
    recs = [[] for _ in range(steps)]
    step_spans: list = []
    t0 = time.perf_counter()
    for j in range(steps):
        one_step(warmup + j, recs[j], step_spans)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    pool.check_errors()
    cache.check_errors()
    cold = None
    if not fused_conv:
        # MALL-cold: the 45 layers' gathers back to back into 45 separate
        # buffers (a 5.8 GiB working set, 23x the 256 MB MALL), then their
        # scatters: every byte of both moves comes from or goes to HBM
        sbufs = [torch.empty((B, *pool.state.shape[2:]), dtype=pool.state.dtype, device=dev)
                 for _ in range(G)]
        cbufs = [torch.empty((B, *pool.conv.shape[2:]), dtype=pool.conv.dtype, device=dev)
                 for _ in range(G)]
        cold = []
        for _ in range(3):
            rec = []
            for g in range(G):
                sp = stamps.span(stream)
                pool.gather(g, slots, out=(sbufs[g], cbufs[g]))
                rec.append(("gather", sp.end(stream)))
            for g in range(G):
                sp = stamps.span(stream)
                pool.scatter(g, slots, sbufs[g], cbufs[g])
                rec.append(("scatter", sp.end(stream)))
            cold.append(rec)
        torch.cuda.synchronize()
        pool.check_errors()
        del sbufs, cbufs
    rec_bytes = 8 * 128 * 128 * 4
    entry = rec_bytes + (0 if fused_conv else 2048 * 4 * 2)
    move_bytes = 2 * B * entry + 4 * B  # one gather or one scatter launch
    # in-place conv: the slot read and written, x in, out, the weights, the slots
    conv_bytes = 2 * B * C * 4 * 2 + 2 * B * C * 2 + C * 4 * 2 + 4 * B
    ratios = counter_ratios("gdn_decode_hbm_counters.md" if fused_conv else
                            "gdn_state_hbm_counters.md")
    g_ms, s_ms, u_ms = _timed(recs, "gather"), _timed(recs, "scatter"), _timed(recs, "update")
    state_s = G * (g_ms + s_ms) / 1e3
    step_s = elapsed / steps
    per_step_state = 4 * G * B * entry + (G * conv_bytes if fused_conv else 0)
    kernels = [
        _kernel_roofline("gdn_decode_gather_kernel<4> (mkv_gdn_decode_gather)" if fused_conv
                         else "state_move_kernel<true> (mkv_state_gather)",
                         move_bytes + (conv_bytes if fused_conv else 0), g_ms,
                         ratios.get("gdn_decode_gather_kernel<4>" if fused_conv
                                    else "state_move_kernel<true>")),
        _kernel_roofline("state_move_kernel<false> (mkv_state_scatter)", move_bytes, s_ms,
                         ratios.get("state_move_kernel<false> fused" if fused_conv
                                    else "state_move_kernel<false>"))]
    res = {
        "metric": ("achieved HBM GB/s (% of 8 TB/s) for GDN decode-step state traffic: "
                   "recurrent slot gather+scatter, conv in place" if fused_conv else
                   "achieved HBM GB/s (% of 8 TB/s) for GDN state slot gather+scatter"),
        "value": round(per_step_state / state_s / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32+bf16",
        "data": "synthetic (seeded ~N(0,1) states, seeded permuted slots)",
        "config": {"workload": (
            "GDN state slots at decode: 45 layers x [8,128,128] fp32 + [2048,4] bf16, "
            "1024-slot pool, batch 256, 60 layers in model order: "
            + ("recurrent gather -> +1 -> scatter and the decode conv (kernel 4) in place on the "
               "conv slots per GDN layer" if fused_conv else
               "gather -> +1 -> scatter per GDN layer")
            + ", decode append per attention layer; seed 105")},
        "state_move_ms_per_step": round(state_s * 1e3, 3),
        "synthetic_update_ms_per_step": round(G * u_ms, 3),
        "step_time": _step_stats(step_spans),
        "pct_of_hbm_peak": round(100 * per_step_state / state_s / 1e9 / HBM_PEAK_GBS, 2),
        "roofline": _roofline_of(sorted(kernels, key=lambda k: -k["mean_launch_us"]),
                                 "gdn_state_hbm_counters.md"),
    }
    if fused_conv:
        res["conv_bytes_per_layer"] = conv_bytes
    if cold is not None:
        cg, cs = _timed(cold[1:], "gather"), _timed(cold[1:], "scatter")
        res["mall_cold"] = {
            "what": ("the 45 gathers back to back into separate buffers (5.8 GiB working set), "
                     "then the 45 scatters, so no byte is served by the 256 MB MALL; mean of "
                     "the last 2 of 3 rounds"),
            "pct_of_hbm_peak": round(100 * 2 * move_bytes / ((cg + cs) / 1e3) / 1e9 / HBM_PEAK_GBS,
                                     2),
            "kernels": [
                _kernel_roofline("state_move_kernel<true> (mkv_state_gather)", move_bytes, cg,
                                 ratios.get("state_move_kernel<true>")),
                _kernel_roofline("state_move_kernel<false> (mkv_state_scatter)", move_bytes, cs,
                                 ratios.get("state_move_kernel<false>"))]}
    if with_cpu:
        from oracle import state as ref
        n = 32
        cpu_pool = pool.state[0, :S].cpu()
        idx = slots[:n].cpu()
        t1 = time.perf_counter()
        x = ref.gather(cpu_pool.unsqueeze(0), 0, idx)
        ref.scatter(cpu_pool.unsqueeze(0), 0, idx, x)
        dt = time.perf_counter() - t1
        res["cpu_baseline"] = {
            "value": round(4 * n * 8 * 128 * 128 * 4 / dt / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"oracle index_select + index_copy_ (torch-CPU) of {n} recurrent "
                       f"states of one layer: {dt*1e3:.1f} ms")}
    return res


def run_plumbing(steps: int, warmup: int, with_cpu: bool) -> dict:
    """1 attention layer, 512 pages x 16, 1 KV head x 256 bf16, 8 prompts of
    randint(1,513) tokens on a seeded shuffled free list: append all prompt
    tokens by slot mapping, gather each back to [len,1,256] (bit-exact check)."""
    from muserve_amd.kv_cache import PagedKVCache, SequenceKVState, prefill_slot_mapping

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(101)
    lens = torch.randint(1, 513, (8,), generator=g).tolist()
    cache = PagedKVCache(512, num_layers=1, dtype=torch.bfloat16, device=dev, verbose=False)
    cache.shuffle_free_list(g)
    seqs = [SequenceKVState() for _ in lens]
    slots = prefill_slot_mapping(cache, seqs, lens)
    T = sum(lens)
    k = torch.randn(T, 1, HEAD_DIM, generator=g).bfloat16().to(dev)
    v = torch.randn(T, 1, HEAD_DIM, generator=g).bfloat16().to(dev)
    width = max(len(s_.page_table) for s_ in seqs)
    bt = torch.zeros(8, width, dtype=torch.int32)
    for b, s_ in enumerate(seqs):
        bt[b, :len(s_.page_table)] = torch.tensor(s_.page_table, dtype=torch.int32)
    bt = bt.to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=dev)
    kout = torch.empty_like(k)
    vout = torch.empty_like(v)

    def one_step():
        cache.append(slots, k, v, layer=0)
        cache.gather(0, bt, sl, out_len=max(lens), cu_out=cu, out=(kout, vout))

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # per-step distribution from a second pass (recording events per step
    # would add host work to this launch-bound loop)
    stamps, spans = Stamps(), []
    stream = torch.cuda.current_stream(dev)
    for _ in range(steps):
        sp = stamps.span(stream)
        one_step()
        spans.append(sp.end(stream))
    torch.cuda.synchronize()
    cache.check_errors()
    exact = bool(torch.equal(kout.view(torch.int16), k.view(torch.int16)) and
                 torch.equal(vout.view(torch.int16), v.view(torch.int16)))
    nbytes = 4 * 512 * T + 8 * T + 4 * 512 * T
    step_s = elapsed / steps
    return {
        "metric": "append + packed gather round trip (us per step; launch-bound, no roofline claim)",
        "value": round(step_s * 1e6, 2), "unit": "us", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "plumbing: 1 layer, 512x16 pool, 8 prompts randint(1,513), seed 101",
                   "tokens": T},
        "step_time": _step_stats(spans),
        "GBps": round(nbytes / step_s / 1e9, 2), "bit_exact_round_trip": exact,
    }


def run_prefix(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Prefix caching at page granularity: 4096 requests (prompts: Zipf(1.1)
    over 64 seeded 4096-token templates + a 64..1024-token random suffix) in
    batches of 256: per batch, SHA-256 page hashes of every prompt, one
    block-manager step (release the previous batch, admit this one: prefix
    lookup, refcounts, allocation with LRU eviction from a 65536-page pool,
    fork + copy-on-write of each partial last page), and the copy-on-write
    page copies (15 layers x K/V x 8 KiB bf16 pages). Timed as a whole trace
    (requests/s and us/request), best of ``steps`` runs on fresh managers."""
    from muserve_amd import _lib
    from muserve_amd.block_manager import BlockManager
    from muserve_amd.kv_cache import PagedKVCache
    from muserve_amd.prefix_hash import page_hashes_range, page_offsets

    dev = torch.device("cuda:0")
    n_req, batch, P = 4096, 256, 65536
    reqs = prefix_requests(n_req, seed=104)
    lens = np.array([len(x) for x in reqs], dtype=np.int64)
    cu_t = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    cu_p = page_offsets(cu_t)
    tokens = torch.from_numpy(np.concatenate(reqs)).to(dev)
    tok_off = torch.from_numpy(cu_t).to(dev)
    page_off = torch.from_numpy(cu_p).to(dev)
    ntok = torch.from_numpy(lens.astype(np.int32)).to(dev)
    hashes = torch.empty(int(cu_p[-1]), dtype=torch.int64, device=dev)
    width = int(-(-lens.max() // 16))
    ops_b = prefix_ops(n_req, batch)
    ops_dev = [torch.tensor(o, dtype=torch.int32, device=dev) for o in ops_b]
    cache = PagedKVCache(P, num_layers=LAYERS, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=torch.bfloat16, device=dev, verbose=False)
    free = np.random.default_rng(104).permutation(P)
    herr = _lib.DeviceErrors(dev)
    stream = torch.cuda.current_stream(dev)

    hash_stream = torch.cuda.Stream(dev)  # default priority, like every stream here
    stamps = Stamps()

    def run_all(bm, rec=None):
        # Page hashing depends only on the prompts and is bound by the longest
        # request's chain of compressions, so all prompts are hashed in one
        # launch on a second stream; the block manager then processes the
        # batches in order, each step waiting for the hashes, each followed by
        # its batch's copy-on-write copies. (Copies on a third stream behind
        # each step, overlapping the next step, did not pay: at full width
        # the copy holds every CU while the step's small kernels wait, and on
        # 128-256 workgroups it is hidden but slows the step's latency-bound
        # kernels by about as much as it saves.)
        with torch.cuda.stream(hash_stream):
            sp = stamps.span(hash_stream) if rec is not None else None
            page_hashes_range(tokens, tok_off, page_off, 0, n_req, hashes, herr)
            if rec is not None:
                rec.append(("hash", sp.end(hash_stream)))
            ready = torch.cuda.Event()
            ready.record(hash_stream)
        stream.wait_event(ready)
        for b, ops in enumerate(ops_dev):
            first = b * batch
            cnt = min(batch, n_req - first)
            sp = stamps.span(stream) if rec is not None else None
            bm.step(ops, hashes, page_off, ntok)
            if rec is not None:
                rec.append(("step", sp.end(stream)))
                sp = stamps.span(stream)
            bm.copy_on_write(cache, first, first + cnt)
            if rec is not None:
                rec.append(("cow", sp.end(stream)))

    for _ in range(warmup):  # whole-trace warm-ups on fresh managers
        run_all(BlockManager(P, n_req, width, dev, free_order=free))
    torch.cuda.synchronize()
    trials = []  # (wall seconds, spans, manager) per whole-trace trial
    for _ in range(max(1, steps)):
        bm = BlockManager(P, n_req, width, dev, free_order=free, evict_log_capacity=1 << 20)
        rec = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run_all(bm, rec)
        torch.cuda.synchronize()
        trials.append((time.perf_counter() - t0, rec, bm))
    walls = np.array([t[0] for t in trials])
    elapsed, rec, bm = trials[int(np.argsort(walls)[len(walls) // 2])]  # the median trial
    bm.check_errors()
    herr.check("page hashes")
    cache.check_errors()
    status = bm.status.cpu().numpy()
    hits = bm.hits.cpu().numpy()
    cow = int((bm.cow_src.cpu().numpy() >= 0).sum())
    ctr = bm.counters()
    n_pages = int(cu_p[-1])
    hash_ms = sum(sp.ms() for lab, sp in rec if lab == "hash")
    step_ms = sum(sp.ms() for lab, sp in rec if lab == "step")
    cow_ms = sum(sp.ms() for lab, sp in rec if lab == "cow")
    page_bytes = 16 * HEAD_DIM * 2
    cow_bytes = cow * 2 * LAYERS * 2 * page_bytes  # read + write, 15 layers x K,V
    us_req = elapsed / n_req * 1e6
    # What a plain contiguous device copy of one batch's copy-on-write bytes
    # takes on this GPU (torch's copy_, same stream and events): the ceiling
    # for a copy of this size, launch and drain included. Each copy takes the
    # next of 16 slices of 2 x ~1 GB buffers, so that (like the pool pages)
    # its source is not in the 256 MB last-level cache from the copy before.
    half = max(1, cow_bytes // len(ops_dev) // 2)
    slices = 16
    src_buf = torch.zeros(slices * half, dtype=torch.uint8, device=dev)
    dst_buf = torch.zeros_like(src_buf)
    spans = []
    for i in range(2 * slices):
        o = (i % slices) * half
        sp = stamps.span(stream)
        dst_buf[o:o + half].copy_(src_buf[o:o + half])
        spans.append(sp.end(stream))
    torch.cuda.synchronize()
    plain_ms = float(np.median([sp.ms() for sp in spans[slices:]]))
    del src_buf, dst_buf
    cow_ratio = counter_ratios("copy_on_write_hbm_counters.md").get("cow")
    res = {
        "metric": "prefix-cache admission: us per request (page hashing + lookup/refcount/"
                  "eviction + copy-on-write)",
        "value": round(us_req, 3), "unit": "us/request", "n_gpus": 1, "steps": max(1, steps),
        "warmup": warmup, "ms_per_step": round(elapsed * 1e3, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "int64 ids / u64 hashes / bf16 pages",
        "data": "synthetic (seeded templates and suffixes)",
        "config": {"workload": ("prefix cache: 4096 requests, Zipf(1.1) over 64 templates of "
                                "4096 random ids + 64..1024-token suffix, batches of 256, "
                                "65536-page pool, 15 layers x 1 KV head x 256 bf16; seed 104")},
        "requests_per_s": round(n_req / elapsed, 1),
        "step_time": {"median_ms": round(float(np.median(walls)) * 1e3, 3),
                      "p10_ms": round(float(np.percentile(walls, 10)) * 1e3, 3),
                      "p90_ms": round(float(np.percentile(walls, 90)) * 1e3, 3),
                      "note": "a step is the whole 4096-request trace on a fresh manager"},
        "pages_hashed_per_s": round(n_pages / (hash_ms / 1e3), 1),
        "admitted": int(((status == 0) | (status == 3)).sum()), "oom": int((status == 1).sum()),
        "page_hit_rate": round(float(hits[status != 1].sum()) / max(1, n_pages), 4),
        "evictions": int(ctr[6]), "cow_copies": cow,
        "phase_ms": {"hash": round(hash_ms, 3), "block_manager": round(step_ms, 3),
                     "cow_copy": round(cow_ms, 3)},
        "hashing": "all prompts hashed in one launch on a second stream before the "
                   "block-manager steps (two lanes per request chain, message schedules "
                   "by a second wave)",
        "roofline": {"kernels": [
            {"kernel": "block_hash_kernel (mkv_block_hash_sha256)", "bound": "integer ALU / latency",
             "note": "the longest request's chain of SHA-256 rounds (two compressions per "
                     "page, ~944 instructions each); no HBM roofline claim",
             "launch_ms": round(hash_ms, 3),
             "GB_hashed_per_s": round(8 * int(cu_t[-1]) / (hash_ms / 1e3) / 1e9, 3)},
            {"kernel": "mkv_bm_step (release run, speculation, group and step kernels)",
             "bound": "latency (a chain of small launches per batch)",
             "us_per_request": round(step_ms * 1e3 / n_req, 3)},
            dict(_kernel_roofline("copy_pages_kernel (mkv_copy_blocks)", cow_bytes / len(ops_dev),
                                  cow_ms / len(ops_dev), cow_ratio),
                 plain_copy_same_bytes={
                     "note": "torch copy_ of one batch's bytes between contiguous slices of 2 x 16 "
                             "batches, each slice cold in cache; median of 16, same events",
                     "us": round(plain_ms * 1e3, 2),
                     "achieved": round(2 * half / (plain_ms / 1e3) / 1e9, 2),
                     "frac": round(2 * half / (plain_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)})]},
    }
    if with_cpu:
        from oracle.blocks import BlockManagerModel
        from oracle.sha import page_hashes as cpu_hashes
        model = BlockManagerModel(P, free.tolist())
        n = batch
        t1 = time.perf_counter()
        for r in range(n):
            model.admit(r, cpu_hashes(reqs[r]), int(lens[r]))
        dt = time.perf_counter() - t1
        gpu_tables = bm.tables[:n].cpu().numpy()
        same = all(gpu_tables[r, :-(-int(lens[r]) // 16)].tolist() == model.reqs[r][0]
                   for r in range(n) if r in model.reqs)
        res["cpu_baseline"] = {
            "value": round(dt / n * 1e6, 3), "unit": "us/request", "cores": 1, "kind": "port",
            "sample": (f"oracle (hashlib incremental page hashes + OrderedDict block manager) for "
                       f"the first batch of {n} requests: {dt:.2f} s; COW copies not included"),
            "gpu_matches_cpu_on_sample": bool(same)}
    return res


Q_HEADS = 4  # query heads per rank over the one KV head (32 / TP 8)


def attn_bytes(lens: np.ndarray, fp8: bool = False) -> float:
    """Algorithmic bytes of one decode-attention launch at lengths ``lens``:
    every cached K and V row once (fp8: 256 code bytes and a 4-byte scale
    each), the table entries, the lengths, q in, out."""
    pages = -(-lens // 16)
    row = HEAD_DIM + 4 if fp8 else ROW
    return float(2 * row * lens.sum() + 4 * pages.sum() + 4 * B + 2 * B * Q_HEADS * ROW)


def attn_cpu_baseline(cache, bt, q, lens_now: np.ndarray, gpu_out, n_seq: int = 16) -> dict:
    """The reference's decode attention (muserve/model/qwen35_layer_v2.py:
    493-502, restated in oracle.attention.reference_bf16: bf16 torch on the
    CPU over K/V gathered from the pages) on the first n_seq sequences of the
    last layer, timed on the host; also checks the GPU output of those
    sequences against the float64 oracle (one bf16 ulp). Over an fp8 pool the
    timed CPU path first dequantises the sequences' pages to bf16
    (oracle.fp8.dequant_rows, as gather_dequant does) and the oracle attends
    over the exact code * scale values, as the fused kernel does."""
    from oracle import attention as att
    from oracle import fp8 as f8

    fp8 = cache.scales is not None
    threads = torch.get_num_threads()
    table = bt.tables.cpu().numpy()[:n_seq]
    lens = lens_now[:n_seq]
    qc = q[LAYERS - 1, :n_seq, 0].cpu()
    if fp8:
        k = cache.cache[LAYERS - 1, 0].cpu().view(torch.uint8)
        v = cache.cache[LAYERS - 1, 1].cpu().view(torch.uint8)
        ks = cache.scales[LAYERS - 1, 0].cpu()
        vs = cache.scales[LAYERS - 1, 1].cpu()
        used = np.unique(np.concatenate([table[b, :-(-int(n) // 16)] for b, n in enumerate(lens)]))
        idx = torch.from_numpy(used.astype(np.int64))
        t0 = time.perf_counter()
        kd = torch.zeros(k.shape, dtype=torch.bfloat16)
        vd = torch.zeros(v.shape, dtype=torch.bfloat16)
        kd[idx] = f8.dequant_rows(k[idx], ks[idx])
        vd[idx] = f8.dequant_rows(v[idx], vs[idx])
        att.reference_bf16(qc, kd, vd, lens, table, HEAD_DIM ** -0.5)
        dt = time.perf_counter() - t0
        want, mass, smax = att.decode_attention(qc.float().numpy(), k.numpy(), v.numpy(), lens,
                                                table, HEAD_DIM ** -0.5, ks.numpy(), vs.numpy(),
                                                stats=True)
        what = "fp8 pages dequantised to bf16, then bf16 torch-CPU attention"
        nbytes = 2 * (HEAD_DIM + 4) * float(lens.sum())
    else:
        k = cache.cache[LAYERS - 1, 0].cpu()
        v = cache.cache[LAYERS - 1, 1].cpu()
        t0 = time.perf_counter()
        att.reference_bf16(qc, k, v, lens, table, HEAD_DIM ** -0.5)
        dt = time.perf_counter() - t0
        want, mass, smax = att.decode_attention(qc.float().numpy(), k.float().numpy(),
                                                v.float().numpy(), lens, table, HEAD_DIM ** -0.5,
                                                stats=True)
        what = "bf16 torch-CPU"
        nbytes = 2 * ROW * float(lens.sum())
    got = gpu_out[:n_seq, 0].float().cpu().numpy().astype(np.float64)
    # one bf16 ulp of the result plus the fp32 evaluation term (scores' error
    # 2^-16 (1 + max|score|) times the attended mass)
    tol = (2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
           + 2.0 ** -16 * (1 + smax[..., None]) * mass)
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s (K/V bytes attended)",
        "cores": threads,
        "kind": "port",
        "sample": (f"reference decode attention ({what}, {threads} threads) over the "
                   f"first {n_seq} sequences of one layer ({int(lens.sum())} cached tokens): "
                   f"{dt:.2f} s"),
        "seconds": round(dt, 3),
        "cpu_model": _cpu_model(),
        "gpu_within_tolerance_of_float64_on_sample": bool((np.abs(got - want) <= tol).all()),
        "tolerance": "1 bf16 ulp of the result + 2^-16 (1 + max|score|) x sum p|v| / sum p",
    }


def run_decode_attn(steps: int, warmup: int, with_cpu: bool, fp8: bool = False) -> dict:
    """Decode step with paged attention instead of the padded gather: per
    layer, append the new token's K/V, then attn_decode for 4 query heads per
    sequence reading the pool through the block tables (same pool, lengths
    and seed as the default workload). fp8: the pool holds e4m3fn codes with
    a scale per token, the append quantises, and attn_decode_fp8 dequantises
    inside the kernel."""
    from muserve_amd.kernels import attention as A
    from muserve_amd.kv_cache import BlockTables, PagedKVCache, SequenceKVState, reserve_tokens

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = context_lengths()
    total_steps = warmup + steps
    pages = int(np.sum(-(-(ctx + total_steps) // 16))) + 64
    log(f"pool: {pages} pages x {LAYERS} layers (ctx sum {int(ctx.sum())}, max {int(ctx.max())})")
    kv_dtype = torch.float8_e4m3fn if fp8 else torch.bfloat16
    cache = PagedKVCache(pages, num_layers=LAYERS, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=kv_dtype, device=dev, verbose=False)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    for l in range(LAYERS):
        if fp8:  # codes of ~N(0,1) rows quantised at absmax ~3.5, scales around 3.5 / 448
            x = torch.empty(cache.cache[l].shape, dtype=torch.bfloat16, device=dev)
            x.normal_(generator=gen)
            cache.cache[l].copy_((x * 128).clamp(-448, 448).to(kv_dtype))
            cache.scales[l].uniform_(0.5 / 128, 1.5 / 128, generator=gen)
            del x
        else:
            cache.cache[l].normal_(generator=gen)
    cache.shuffle_free_list(torch.Generator().manual_seed(SEED))
    seqs = [SequenceKVState() for _ in range(B)]
    for s, n in zip(seqs, ctx):
        reserve_tokens(cache, s, int(n))
    width = int(-(-(int(ctx.max()) + total_steps) // 16))
    bt = BlockTables(cache, seqs, max_pages=width)
    kin = torch.empty(total_steps, LAYERS, B, 1, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vin = torch.empty_like(kin)
    kin.normal_(generator=gen)
    vin.normal_(generator=gen)
    q = torch.empty(LAYERS, B, 1, Q_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    q.normal_(generator=gen)
    out = torch.empty(LAYERS, B, 1, Q_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    max_len = int(ctx.max()) + total_steps
    stream = torch.cuda.current_stream(dev)
    stamps = Stamps()

    def one_step(i: int, rec=None, steps_rec=None):
        step = stamps.span(stream) if steps_rec is not None else None
        slots = bt.decode_step()
        for l in range(LAYERS):
            cache.append(slots, kin[i, l], vin[i, l], layer=l)
            kp, vp = cache.get_kv_by_layer(l)
            sp = stamps.span(stream) if rec is not None else None
            if fp8:
                A.attn_decode_fp8(q[l], kp, vp, cache.scales[l, 0], cache.scales[l, 1],
                                  bt.seq_lens, bt.tables, max_seqlen=max_len, out=out[l])
            else:
                A.attn_decode(q[l], kp, vp, bt.seq_lens, bt.tables, max_seqlen=max_len,
                              out=out[l])
            if rec is not None:
                rec.append(("attn", sp.end(stream)))
        if steps_rec is not None:
            steps_rec.append(step.end(stream))

    log(f"warmup {warmup} steps")
    for i in range(warmup):
        one_step(i)
    torch.cuda.synchronize()
    cache.check_errors()
    A.check_errors(dev)

    lens0 = bt._lens.copy()
    attn_total = step_total = 0.0
    stored = HEAD_DIM + 4 if fp8 else ROW  # bytes the append writes per K or V row
    for j in range(steps):
        ab = attn_bytes(lens0 + j + 1, fp8)
        attn_total += ab
        step_total += LAYERS * (ab + 2 * B * ROW + 2 * B * stored + 8 * B)  # + the append
    recs = [[] for _ in range(steps)]
    step_spans: list = []
    log(f"timing {steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for j in range(steps):
        one_step(warmup + j, recs[j], step_spans)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    cache.check_errors()
    A.check_errors(dev)
    mean_attn_s = _timed(recs, "attn") / 1e3
    mean_attn_bytes = attn_total / steps
    ratio = counter_ratios("decode_attention_hbm_counters.md").get("attn_fp8" if fp8 else "attn")
    step_s = elapsed / steps
    value = step_total / elapsed / 1e9
    achieved = mean_attn_bytes / mean_attn_s / 1e9
    res = {
        "metric": ("achieved HBM GB/s (% of 8 TB/s) for KV append + paged decode attention"
                   + (" over an fp8 pool" if fp8 else "") + "; decode step µs @ batch 256"),
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp8 e4m3fn KV with fp32 scales, bf16 q/out (fp32 softmax and accumulation)"
                  if fp8 else "bf16 (fp32 softmax and accumulation)"),
        "data": "synthetic (seeded ~N(0,1) q/K/V, seeded log-normal context lengths)",
        "config": {
            "workload": ("decode-step KV append + paged decode attention on one TP rank: 15 "
                         "attention layers, batch 256, 4 query heads over 1 KV head x 256, "
                         + ("fp8 e4m3fn KV (per-token fp32 scales, quantised on append, "
                            "dequantised in the kernel)" if fp8 else "bf16")
                         + ", 16-token pages, ctx lognormal(median 4096, sigma 1.0, clip "
                         "1..32768), seed 102"),
            "batch": B, "layers": LAYERS, "q_heads": Q_HEADS, "kv_heads": 1, "head_dim": HEAD_DIM,
            "ctx_sum_start": int(lens0.sum()), "ctx_max_start": int(lens0.max()),
        },
        "decode_step_us": round(step_s * 1e6, 1),
        "step_time": _step_stats(step_spans),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(B / step_s, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": ("mkv_decode_attention_fp8 = attn_span_kernel<4, true> + "
                       "attn_merge_kernel<4>" if fp8 else
                       "mkv_decode_attention_bf16 = attn_span_kernel<4, false> + "
                       "attn_merge_kernel<4>"),
            "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": round(ratio * mean_attn_bytes) if ratio else None,
            "traffic_to_algorithmic": ratio,
            "traffic_source": ("rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 (scales from a 1 GiB "
                               "copy), profiles/decode_attention_hbm_counters.md"),
            "mean_launch_us": round(mean_attn_s * 1e6, 2),
            "algorithmic_bytes_per_launch": round(mean_attn_bytes),
            "flop_per_launch": round(4 * Q_HEADS * HEAD_DIM * float((lens0 + steps).sum())),
        },
    }
    if with_cpu:
        log("cpu baseline (reference decode attention on a sample)")
        res["cpu_baseline"] = attn_cpu_baseline(cache, bt, q, bt._lens.copy(), out[LAYERS - 1])
    return res


SCHED_SEED = 106
SCHED_BATCH = 256          # muserve/config.py:32-33 MAX_RUNNING_REQUESTS / MAX_DECODE_BATCH
SCHED_MAX_PROMPT = 8192
SCHED_MAX_NEW = 512
SCHED_PHASE_EVERY = 4      # serving steps per step with per-phase event spans


def sched_requests(n: int, seed: int = SCHED_SEED) -> tuple[np.ndarray, np.ndarray]:
    """Prompt lengths lognormal(median 1024, sigma 1) clipped to [16, 8192];
    output lengths uniform in [32, 512]."""
    rng = np.random.default_rng(seed)
    prompts = np.clip(np.round(rng.lognormal(np.log(1024.0), 1.0, n)), 16,
                      SCHED_MAX_PROMPT).astype(np.int64)
    return prompts, rng.integers(32, SCHED_MAX_NEW + 1, n)


def run_sched(steps: int, warmup: int, with_cpu: bool, fp8: bool = False,
              hybrid: bool = False, serial_prefill: bool = False, prefix: bool = False) -> dict:
    """Continuous-batching serving steps on one TP rank, driven by the
    scheduler's step plan: a backlog of requests, at most 256 running, a
    4096-token chunked-prefill budget per step (muserve/config.py:33,40).
    Per step: plan_step (one upload + one mkv_step_plan launch: slot mapping,
    positions, cu_seqlens, per-entry block tables), then per attention layer
    the append of every scheduled token's K/V through the slot mapping and
    paged decode attention (4 query heads) for the decode entries through the
    plan's tables; complete_step retires requests at their output length.
    The warmup fills the batch; the timed steps run with it full.
    fp8: an e4m3fn pool (quantise on append, dequantise inside attention).
    hybrid: the 60-layer stack in model order; each of the 45 GDN layers moves
    the scheduled requests' state slots (a request's batch row is its slot,
    zeroed at admission): decode entries through the fused recurrent gather +
    in-place decode conv, prefill entries through a gather of both states,
    then a scatter of the recurrent states back (the GDN recurrence itself is
    model math and is not run).
    prefix: the prefix-cache configuration's prompts (Zipf(1.1) over 64
    templates of 4096 ids + a 64..1024-token suffix) served with prefix reuse:
    a block manager owns most of the pool, admissions hash their prompts on
    the GPU and skip the cached pages' tokens."""
    from muserve_amd.kernels import attention as A
    from muserve_amd.kv_cache import PagedKVCache
    from muserve_amd.scheduler import ContinuousBatchScheduler, InferenceRequest
    from muserve_amd.state_pool import StatePool, gdn_ordinal

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    max_seq = SCHED_MAX_PROMPT + SCHED_MAX_NEW
    width = -(-max_seq // 16)
    pages = SCHED_BATCH * width + 64  # every running request can reach max_seq: no OOM
    n_req = 4096
    prompts, outs = sched_requests(n_req)
    bm = None
    if prefix:
        from muserve_amd.block_manager import BlockManager
        token_ids = prefix_requests(n_req, seed=104)
        prompts = np.array([len(x) for x in token_ids], dtype=np.int64)
        # block manager: every running request's shareable pages plus the
        # 64 templates' pages (16,384) cached; private: a tail page and the
        # decode pages of every running request
        bm_pages = SCHED_BATCH * int(-(-prompts.max() // 16)) + 64 * 4096 // 16
        pages = bm_pages + SCHED_BATCH * (SCHED_MAX_NEW // 16 + 2) + 64
    kv_dtype = torch.float8_e4m3fn if fp8 else torch.bfloat16
    cache = PagedKVCache(pages, num_layers=LAYERS, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=kv_dtype, device=dev, verbose=False)
    cache.shuffle_free_list(torch.Generator().manual_seed(SCHED_SEED))
    if prefix:
        bm = BlockManager(bm_pages, 2 * SCHED_BATCH, width, dev,
                          free_order=np.random.default_rng(SCHED_SEED).permutation(bm_pages))
    free0 = list(cache._free_pages)
    chunk = 4096
    gen = torch.Generator(device=dev).manual_seed(SCHED_SEED)
    pool = None
    if hybrid:
        pool = StatePool(num_layers=45, num_slots=SCHED_BATCH, device=dev)
        pool.state.normal_(generator=gen)
        pool.conv.normal_(generator=gen)
    s = ContinuousBatchScheduler(max_batch_size=SCHED_BATCH, max_seq_len=max_seq, kv_cache=cache,
                                 chunked_prefill_size=chunk, state_pool=pool, block_manager=bm)
    # pages several running requests may read: the block manager's cached
    # prompt pages [0, bm_pages); the private tail and decode pages lie above
    shared = bm.num_pages if bm is not None else 0
    for i in range(n_req):
        ids = token_ids[i].tolist() if prefix else [0] * int(prompts[i])
        s.add_request(InferenceRequest(request_id=str(i), input_ids=ids,
                                       max_new_tokens=int(outs[i])))
    max_t = SCHED_BATCH + chunk
    kin = torch.empty(LAYERS, max_t * HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vin = torch.empty_like(kin)
    kin.normal_(generator=gen)
    vin.normal_(generator=gen)
    q = torch.empty(LAYERS, SCHED_BATCH, 1, Q_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    q.normal_(generator=gen)
    out = torch.empty_like(q)
    # the prefill chunks' queries (bf16 pools: their attention over the pool)
    qp = torch.empty(chunk * Q_HEADS * HEAD_DIM, dtype=torch.bfloat16, device=dev).normal_(
        generator=gen)
    outp = torch.empty_like(qp)
    if hybrid:
        C = pool.conv.shape[2]
        xin = torch.randn(45, SCHED_BATCH, C, generator=gen, device=dev).bfloat16()
        wconv = (0.5 * torch.randn(45, C, 1, 4, generator=gen, device=dev)).bfloat16()
        sbuf = torch.empty((SCHED_BATCH, *pool.state.shape[2:]), dtype=pool.state.dtype,
                           device=dev)
        cbuf = torch.empty((SCHED_BATCH, *pool.conv.shape[2:]), dtype=pool.conv.dtype, device=dev)
        cout = torch.empty(SCHED_BATCH, C, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    # the prefill chunks' attention (MFMA-bound) runs on a second stream of
    # default priority, beside the decode attention (HBM-bound): both read
    # the layer's pool after its append and write separate outputs; the
    # streams join at the end of the step, before the plan buffers are reused
    side = None if serial_prefill else torch.cuda.Stream(dev)
    # fp8 pools: the prefill entries' context windows are dequantised to bf16
    # by the packed block-table gather, then attended by attn_prefill over
    # contiguous K/V (the reference's fp8 chunked-prefill flow)
    deq = {"rows": 0, "k": None, "v": None}
    stamps = Stamps()
    log(f"pool: {pages} pages x {LAYERS} layers ({kv_dtype}); {n_req} queued requests "
        f"(prompt median {int(np.median(prompts))}, max {int(prompts.max())})"
        + ("; 45 GDN layers x 256 state slots" if hybrid else ""))

    first_slots = []  # slot mappings of the first steps, checked against the oracle
    layer_order = list(range(60)) if hybrid else [4 * l + 3 for l in range(LAYERS)]

    def one_step(rec=None, host=None, info=None):
        t0 = time.perf_counter()
        plan = s.plan_host()
        if host is not None:
            host.append(time.perf_counter() - t0)
        sp = stamps.span(stream) if rec is not None else None
        s.launch_plan(plan)
        if rec is not None:
            rec.append(("plan", sp.end(stream)))
        T, nd, n = plan.num_tokens, plan.num_decode, plan.num_entries
        if len(first_slots) < 8:
            first_slots.append(plan.slot_mapping.cpu().tolist())
        # the decode half's lengths after this step's append (host copy of
        # what the kernel writes), for the byte count
        ent = plan.upload[:8 * nd].reshape(nd, 8)
        lens = ent[:, 1] + ent[:, 2]
        if n > nd:
            # decode entries hold one token each; int32 once per step, as the
            # attention kernels take it
            cu_pre = (plan.cu_seqlens[nd:] - nd).to(torch.int32)
            max_chunk = max(c for _, _, c in plan.prefill)
            max_ctx = max(st + c for _, st, c in plan.prefill)
            if fp8:  # packed bf16 windows: sequence b's context at cu_ctx[b]
                ctx_rows = sum(st + c for _, st, c in plan.prefill)
                cu_ctx = torch.zeros(n - nd + 1, dtype=torch.int32, device=dev)
                cu_ctx[1:] = torch.cumsum(plan.seq_lens[nd:], 0)
                if deq["rows"] < ctx_rows:  # grown, never freed (the side stream reads it)
                    rows = max(ctx_rows, 2 * deq["rows"])
                    deq["k"] = torch.empty(rows, 1, HEAD_DIM, dtype=torch.bfloat16, device=dev)
                    deq["v"] = torch.empty_like(deq["k"])
                    deq.setdefault("kept", []).append((deq["k"], deq["v"]))
                    deq["rows"] = rows
        for layer in layer_order:
            if layer % 4 != 3:  # a GDN layer: the scheduled requests' state slots
                g = gdn_ordinal(layer)
                sp = stamps.span(stream) if rec is not None else None
                if nd:
                    pool.decode_gather(g, plan.rows[:nd], xin[g, :nd], wconv[g],
                                       state_out=sbuf[:nd], conv_out=cout[:nd])
                if n > nd:
                    pool.gather(g, plan.rows[nd:], out=(sbuf[nd:n], cbuf[nd:n]))
                pool.scatter(g, plan.rows, sbuf[:n])
                if rec is not None:
                    rec.append(("gdn", sp.end(stream)))
                continue
            l = layer // 4
            sp = stamps.span(stream) if rec is not None else None
            cache.append(plan.slot_mapping, kin[l, :T * HEAD_DIM].view(T, 1, HEAD_DIM),
                         vin[l, :T * HEAD_DIM].view(T, 1, HEAD_DIM), layer=l)
            if rec is not None:
                rec.append(("append", sp.end(stream)))
            if side is not None and n > nd:
                appended = stamps.record(stream)
            if nd:
                kp, vp = cache.get_kv_by_layer(l)
                sp = stamps.span(stream) if rec is not None else None
                if fp8:
                    A.attn_decode_fp8(q[l, :nd], kp, vp, cache.scales[l, 0], cache.scales[l, 1],
                                      plan.seq_lens[:nd], plan.block_tables[:nd], out=out[l, :nd],
                                      shared_pages=shared)
                else:
                    A.attn_decode(q[l, :nd], kp, vp, plan.seq_lens[:nd], plan.block_tables[:nd],
                                  out=out[l, :nd], shared_pages=shared)
                if rec is not None:
                    rec.append(("attn", sp.end(stream)))
            if n > nd:  # the prefill chunks attend to their prefix and themselves
                kp, vp = cache.get_kv_by_layer(l)
                tp = T - nd
                qv = qp[:tp * Q_HEADS * HEAD_DIM].view(tp, Q_HEADS, HEAD_DIM)
                ov = outp[:tp * Q_HEADS * HEAD_DIM].view(tp, Q_HEADS, HEAD_DIM)
                ps = stream
                if side is not None:
                    stamps.wait(side, appended)
                    ps = side
                with torch.cuda.stream(ps):
                    if fp8:
                        sp = stamps.span(ps) if rec is not None else None
                        kd, vd = deq["k"][:ctx_rows], deq["v"][:ctx_rows]
                        cache.gather(l, plan.block_tables[nd:], plan.seq_lens[nd:],
                                     out_len=max_ctx, cu_out=cu_ctx, out=(kd, vd))
                        if rec is not None:
                            rec.append(("prefill_dequant", sp.end(ps)))
                    sp = stamps.span(ps) if rec is not None else None
                    if fp8:
                        A.attn_prefill(qv, kd, vd, cu_pre, cu_ctx, max_chunk, max_ctx, out=ov)
                    else:
                        A.attn_prefill_paged(qv, kp, vp, cu_pre, plan.seq_lens[nd:],
                                             plan.block_tables[nd:], max_chunk,
                                             max_seqlen_k=max_ctx, out=ov)
                if rec is not None:
                    rec.append(("prefill_attn", sp.end(ps)))
        if side is not None and n > nd:
            stamps.wait(stream, stamps.record(side))
        if info is not None:
            info.append((T, nd, len(plan.prefill), lens, plan.block_tables.shape[1], n,
                         [(st, c) for _, st, c in plan.prefill]))
        s.complete_step(plan)

    log(f"warmup {warmup} steps")
    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    cache.check_errors()
    s.check_errors()
    A.check_errors(dev)
    if pool is not None:
        pool.check_errors()
    recs = [[] for _ in range(steps)]
    host: list[float] = []
    info: list = []
    log(f"timing {steps} steps ({s.num_running} running, {s.num_prefilling} prefilling, "
        f"{s.num_waiting} waiting)")
    skipped0 = s.prefix_skipped
    step_spans: list = []
    t0 = time.perf_counter()
    for j in range(steps):
        step = stamps.span(stream)
        # the per-phase spans on every SCHED_PHASE_EVERY-th step: each is two
        # event records on the host, which a step of ~50 short launches feels
        one_step(recs[j] if j % SCHED_PHASE_EVERY == 0 else None, host, info)
        step_spans.append(step.end(stream))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    cache.check_errors()
    s.check_errors()
    A.check_errors(dev)
    if pool is not None:
        pool.check_errors()
    tokens = sum(x[0] for x in info)
    decode_tokens = sum(x[1] for x in info)
    row_kv = HEAD_DIM + 4 if fp8 else ROW  # bytes of one cached K or V row
    attn_b = append_b = gdn_b = 0.0
    st_b = pool.state[0, 0].numel() * 4 if hybrid else 0
    cv_b = pool.conv[0, 0].numel() * 2 if hybrid else 0
    for T, nd, _, lens, w, n, _pre in info:
        if nd:
            ln = lens.astype(np.int64)
            attn_b += LAYERS * float(2 * row_kv * ln.sum() + 4 * (-(-ln // 16)).sum() + 4 * nd
                                     + 2 * nd * Q_HEADS * ROW)
        append_b += LAYERS * float(2 * T * ROW + 2 * T * row_kv + 8 * T)
        if hybrid:  # decode: state gather + conv in place (+ x, out); prefill: both gathered;
            # then every entry's state scattered back
            C = pool.conv.shape[2]
            gdn_b += 45 * float(nd * (2 * st_b + 2 * cv_b + 4 * C + 8)
                                + (n - nd) * (2 * st_b + 2 * cv_b + 4) + n * (2 * st_b + 4))
    attn_launches = LAYERS * sum(1 for x in info if x[1])
    # prefill attention: 4 x D flops per (query head, visible key) pair x 4 heads
    pre_pairs = sum(c * st + c * (c + 1) // 2 for x in info for st, c in x[6])
    pre_flops = LAYERS * 4.0 * HEAD_DIM * Q_HEADS * pre_pairs
    pre_ms = _timed(recs, "prefill_attn")
    attn_ms = _timed(recs, "attn")
    plan_ms = _timed(recs, "plan")
    append_ms = _timed(recs, "append")
    step_s = elapsed / steps
    value = (attn_b + append_b + gdn_b) / elapsed / 1e9
    achieved = attn_b / attn_launches / (attn_ms / 1e3) / 1e9
    ratio = None if hybrid else counter_ratios("sched_serving_kernel_trace.md").get(
        "attn_fp8" if fp8 else ("attn_prefix" if prefix else "attn"))
    kernel = ("mkv_decode_attention_fp8 = attn_span_kernel<4, true> + attn_merge_kernel<4>"
              if fp8 else
              "mkv_decode_attention_bf16 = attn_span_kernel<4, false> + attn_merge_kernel<4>")
    res = {
        "metric": ("achieved HBM GB/s (% of 8 TB/s) of continuous-batching serving steps "
                   "(scheduler step plan + KV append + paged decode attention"
                   + ("" if fp8 else " + paged prefill attention")
                   + (" + GDN state slot moves" if hybrid else "") + "); step µs"),
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp8 e4m3fn KV with fp32 scales, bf16 q/out (fp32 softmax and accumulation)"
                  if fp8 else "bf16 (fp32 softmax and accumulation)")
                 + ("; fp32 recurrent / bf16 conv GDN states" if hybrid else ""),
        "data": ("synthetic (seeded ~N(0,1) q/K/V; seeded lognormal prompt lengths, uniform "
                 "output lengths; a sampled token is a placeholder)"),
        "config": {
            "workload": ("continuous-batching serving on one TP rank: 4096 queued requests, "
                         + ("prompts Zipf(1.1) over 64 templates of 4096 random ids + a "
                            "64..1024-token suffix (seed 104) with prefix reuse through the "
                            "block manager" if prefix else
                            "prompts lognormal(median 1024, sigma 1, clip 16..8192)")
                         + ", outputs uniform 32..512 tokens, at most 256 running, 4096-token chunked "
                         "prefill budget per step; 15 attention layers, 1 KV head x 256, "
                         + ("fp8 e4m3fn" if fp8 else "bf16") + " pool of 16-token pages, "
                         "4 query heads"
                         + ("; 60 layers in model order with 45 GDN layers' state slots "
                            "([8,128,128] fp32 + [2048,4] bf16 per request)" if hybrid else "")
                         + "; seed 106"),
            "max_batch": SCHED_BATCH, "chunked_prefill_size": chunk, "layers": LAYERS,
            "kv_heads": 1, "head_dim": HEAD_DIM, "q_heads": Q_HEADS, "pool_pages": pages,
            "gdn_layers": 45 if hybrid else 0,
        },
        "step_time": _step_stats(step_spans),
        "tokens_per_s": round(tokens / elapsed, 1),
        "decode_tokens_per_s": round(decode_tokens / elapsed, 1),
        "prefill_tokens_per_s": round((tokens - decode_tokens) / elapsed, 1),
        "mean_entries": {"decode": round(decode_tokens / steps, 1),
                         "prefill_chunks": round(sum(x[2] for x in info) / steps, 2),
                         "tokens": round(tokens / steps, 1)},
        "plan_device_us": round(plan_ms * 1e3, 2),
        "plan_device_note": "upload of the step records + the mkv_step_plan launch (events)",
        "plan_host_us": round(float(np.mean(host)) * 1e6, 1),
        "plan_host_us_p90": round(float(np.percentile(host, 90)) * 1e6, 1),
        "append_us_per_layer": round(append_ms * 1e3, 2),
        "attn_us_per_layer": round(attn_ms * 1e3, 2),
        "roofline": {
            "bound": "hbm", "kernel": kernel,
            "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": round(ratio * attn_b / attn_launches) if ratio else None,
            "traffic_to_algorithmic": ratio,
            "traffic_source": ("rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 of the same kernel in "
                               "this workload, profiles/sched_serving_kernel_trace.md"
                               if ratio else None),
            "mean_launch_us": round(attn_ms * 1e3, 2),
            "algorithmic_bytes_per_launch": round(attn_b / attn_launches),
            **({"note": "algorithmic bytes count a page shared through prefix reuse once per "
                        "sequence reading it; those reads mostly hit in L2 or the last-level "
                        "cache, so achieved can pass the HBM peak, and HBM traffic is the "
                        "traffic field"} if prefix else {}),
            # with the prefill attention on a second stream the two kernels
            # share the GPU, and the event span above times the decode
            # attention while it does: not a per-kernel figure (run with
            # --serial-prefill for that)
            "concurrent": side is not None,
        },
    }
    if side is not None:
        res["roofline"]["note"] = ("measured while the prefill attention ran beside it on a "
                                   "second stream; the per-kernel fraction comes from "
                                   "--serial-prefill, the step-level figure is `value`")
    if pre_pairs:
        n_pre = LAYERS * sum(1 for x in info if x[6])
        pre_tf = pre_flops / n_pre / (pre_ms / 1e3) / 1e12
        res["prefill_attn_us_per_layer"] = round(pre_ms * 1e3, 2)
        res["prefill_attn_TFLOPs"] = round(pre_tf, 2)
        if fp8:
            res["prefill_dequant_us_per_layer"] = round(_timed(recs, "prefill_dequant") * 1e3, 2)
        res["roofline_prefill_attention"] = {
            "bound": "mfma", "kernel": "prefill_attn_kernel + prefill_merge_kernel "
            + ("(mkv_prefill_attention_bf16 over the dequantised contiguous windows, key ranges "
               "split)" if fp8 else "(mkv_prefill_attention_bf16, paged, key ranges split)"),
            "achieved": round(pre_tf, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(pre_tf / MFMA_BF16_PEAK_TFLOPS, 4), "mean_launch_us": round(pre_ms * 1e3, 2),
            "flop_per_launch": round(pre_flops / n_pre), "concurrent": side is not None,
            "stream": "main, after the decode attention" if side is None else
                      "second stream, concurrent with the decode attention (launch time "
                      "measured while sharing the GPU)"}
    if hybrid:
        gdn_ms = _timed(recs, "gdn")
        res["gdn_us_per_layer"] = round(gdn_ms * 1e3, 2)
        res["gdn_GBps"] = round(gdn_b / steps / 45 / (gdn_ms / 1e3) / 1e9, 2)
    if prefix:
        skipped = s.prefix_skipped - skipped0
        prompt_tok = tokens - decode_tokens + skipped  # prefill tokens computed + served
        res["prefix"] = {
            "block_manager_pages": bm.num_pages, "private_pages": pages - bm.num_pages,
            "prompt_tokens_skipped": int(skipped),
            "prompt_tokens_computed": int(tokens - decode_tokens),
            "skipped_fraction": round(skipped / max(1, prompt_tok), 4),
            "prompt_tokens_per_s_incl_skipped": round(prompt_tok / elapsed, 1),
            "evictions": int(bm.counters()[6]),
            # rounds with admits (warm-up included) whose results were read
            # after the many-CU half / after the one-workgroup kernels (a
            # round of at most 8 ops is the step kernel alone: late)
            "block_manager_rounds_read": {"early": s.bm_early_rounds, "late": s.bm_late_rounds},
            "note": ("the timed steps' prompt tokens found in cached pages (never computed or "
                     "appended); plan_host_us includes the block-manager round "
                     "(mkv_bm_step_begin/_end on a side stream: the step's releases and "
                     "admits) and the wait for its results; prompts are hashed on the side "
                     "stream when they are queued"),
        }
    if with_cpu and not prefix:
        log("cpu baseline (scheduler oracle: per-token page bookkeeping of the same trace)")
        res["cpu_baseline"] = sched_cpu_baseline(prompts, outs, pages, free0, chunk, max_seq,
                                                 first_slots, warmup, steps)
    return res


def sched_cpu_baseline(prompts, outs, pages, free0, chunk, max_seq, first_slots, warmup: int,
                       steps: int, budget_s: float = 20.0) -> dict:
    """The scheduler oracle (per-token SequenceKVState bookkeeping with
    alloc_pages(1), muserve/kv_cache.py:133-158, and per-entry page-table
    lists) planning the same trace from its start: the warmup steps, then
    the timed steps (as many as fit in budget_s seconds of host time); its
    first steps' slot mappings are compared with the GPU's."""
    from oracle import paged as pg
    from oracle import sched as S

    m = S.ChunkedSchedulerModel(SCHED_BATCH, chunk, pg.PoolModel(pages, free0), max_seq)
    for i, (n, g) in enumerate(zip(prompts, outs)):
        m.add(S.Req(str(i), int(n), int(g)))
    same = True
    t_all = t_timed = 0.0
    n = tokens = timed = 0
    while n < warmup + steps and t_all < budget_s:
        t0 = time.perf_counter()
        out = m.step()
        dt = time.perf_counter() - t0
        t_all += dt
        if n < len(first_slots):
            same = same and out["slots"] == first_slots[n]
        if n >= warmup:
            t_timed += dt
            tokens += len(out["slots"])
            timed += 1
        n += 1
        m.complete()
    return {"value": round(t_timed / timed * 1e6, 1) if timed else None,
            "unit": "us per step (plan only)", "cores": 1, "kind": "port",
            "sample": (f"scheduler oracle (pure Python, 1 thread) planning the same trace: "
                       f"{warmup} warmup steps, then {timed} of the timed steps "
                       f"({tokens} tokens): {t_timed:.1f} s of {t_all:.1f} s"),
            "gpu_matches_cpu_on_first_steps": bool(same),
            "steps_compared": min(n, len(first_slots))}


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (no sparsity)


def run_prefill_attn(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Varlen causal prefill attention (attn_prefill, the reference's
    flash_attn_varlen_func interface): 8 prompts of 4096 tokens, 4 query heads
    over 1 KV head of 256, bf16, 15 attention layers per step (each layer its
    own q/k/v). MFMA-bound: the roofline is the bf16 dense peak."""
    from muserve_amd.kernels import attention as A
    from oracle import attention as att

    dev = torch.device("cuda:0")
    nseq, L = 8, 4096
    T = nseq * L
    gen = torch.Generator(device=dev).manual_seed(107)
    q = torch.empty(LAYERS, T, Q_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev).normal_(
        generator=gen)
    k = torch.empty(LAYERS, T, 1, HEAD_DIM, dtype=torch.bfloat16, device=dev).normal_(
        generator=gen)
    v = torch.empty_like(k).normal_(generator=gen)
    out = torch.empty(T, Q_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    cu = torch.arange(0, T + 1, L, dtype=torch.int32, device=dev)
    pairs = nseq * L * (L + 1) // 2
    flops = 4.0 * HEAD_DIM * Q_HEADS * pairs  # QK^T and PV, 2 flop per multiply-add each
    stream = torch.cuda.current_stream(dev)
    stamps = Stamps()

    def one_step(rec=None):
        for l in range(LAYERS):
            sp = stamps.span(stream) if rec is not None else None
            A.attn_prefill(q[l], k[l], v[l], cu, cu, L, L, out=out)
            if rec is not None:
                rec.append(("attn", sp.end(stream)))

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    A.check_errors(dev)
    recs = [[] for _ in range(steps)]
    t0 = time.perf_counter()
    for j in range(steps):
        one_step(recs[j])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    A.check_errors(dev)
    ms = _timed(recs, "attn")
    achieved = flops / (ms / 1e3) / 1e12
    step_s = elapsed / steps
    # the last layer's output on the first 64 tokens of sequence 0 (causal: they
    # depend on its first 64 keys only) against the float64 oracle
    n = 64
    want, mass = att.prefill_attention(q[LAYERS - 1, :n].float().cpu().numpy(),
                                       k[LAYERS - 1, :n].float().cpu().numpy(),
                                       v[LAYERS - 1, :n].float().cpu().numpy(), [0, n],
                                       HEAD_DIM ** -0.5, True, cu_k=[0, n], stats=True)
    got = out[:n].float().cpu().numpy().astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    sample_ok = bool((np.abs(got - want) <= ulp + 2.0 ** -8 * mass).all())
    res = {
        "metric": "varlen causal prefill attention TFLOP/s (bf16 MFMA)",
        "value": round(achieved, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 (fp32 softmax and accumulation, bf16 probabilities for P V)",
        "data": "synthetic (seeded ~N(0,1) q/K/V)",
        "config": {"workload": ("varlen causal prefill attention: 8 prompts x 4096 tokens, 4 query "
                                "heads over 1 KV head x 256, bf16, 15 attention layers; seed 107"),
                   "sequences": nseq, "tokens": L, "layers": LAYERS},
        "attention_us_per_layer": round(ms * 1e3, 2),
        "gpu_matches_oracle_on_sample": sample_ok,
        "roofline": {"bound": "mfma", "kernel": "prefill_attn_kernel (mkv_prefill_attention_bf16)",
                     "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None, "mean_launch_us": round(ms * 1e3, 2),
                     "flop_per_launch": flops,
                     "flop_note": "4 x head_dim x query heads per visible (query, key) pair"},
    }
    if with_cpu:
        import torch.nn.functional as F
        m = 1024
        qc = q[0, :m].float().cpu().permute(1, 0, 2).contiguous()
        kc = k[0, :m].float().cpu().repeat_interleave(Q_HEADS, 1).permute(1, 0, 2).contiguous()
        vc = v[0, :m].float().cpu().repeat_interleave(Q_HEADS, 1).permute(1, 0, 2).contiguous()
        reps = 0
        t1 = time.perf_counter()
        while time.perf_counter() - t1 < 10.0 and reps < 200:
            F.scaled_dot_product_attention(qc, kc, vc, is_causal=True)
            reps += 1
        dt = (time.perf_counter() - t1) / reps
        res["cpu_baseline"] = {
            "value": round(4.0 * HEAD_DIM * Q_HEADS * (m * (m + 1) // 2) / dt / 1e12, 4),
            "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"torch CPU scaled_dot_product_attention (fp32, causal) on one "
                       f"{m}-token sequence, {reps} runs: {dt * 1e3:.1f} ms each")}
    return res


HOST_LINK_PEAK_GBS = 64.0  # PCIe Gen5 x16, per direction (published)


def run_offload(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Prefix-cache host tier (muserve/model/prefix_cache.py:36-44 replaced):
    per step, store one 32K-token prefix entry of one rank into pinned host
    memory, then restore it. The entry holds:
    - the hidden state of every prefill token, [32768, 4096] bf16, as the
      reference stores it;
    - the 45 GDN states, [1, 8, 128, 128] fp32;
    - the prefix's KV pages in all 15 attention layers (2048 pages, which the
      reference does not keep).
    The restore (lookup_kv) writes the KV into fresh pool pages. A second
    restore without KV times the reference's content alone."""
    from muserve_amd.kv_cache import PagedKVCache
    from muserve_amd.model.prefix_cache import PrefixCache

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, hidden_size, n_gdn = 32768, 4096, 45
    n_pages = T // 16
    cache = PagedKVCache(2 * n_pages + 64, num_layers=LAYERS, kv_heads=1, head_dim=HEAD_DIM,
                         dtype=torch.bfloat16, device=dev, verbose=False)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    cache.cache.normal_(generator=gen)
    cache.shuffle_free_list(torch.Generator().manual_seed(SEED))
    pages = cache.alloc_pages(n_pages)
    hidden = torch.empty(T, hidden_size, dtype=torch.bfloat16, device=dev).normal_(generator=gen)
    states = [torch.empty(1, 8, 128, 128, device=dev).normal_(generator=gen)
              for _ in range(n_gdn)]
    dense_bytes = hidden.numel() * 2 + n_gdn * 8 * 128 * 128 * 4
    kv_bytes = LAYERS * 2 * n_pages * 16 * HEAD_DIM * 2
    entry_bytes = dense_bytes + kv_bytes
    pc = PrefixCache(max_entries=2, host_bytes=2 * entry_bytes + (64 << 20))
    ids_base = torch.arange(T + 16, dtype=torch.int64)
    stream = torch.cuda.current_stream(dev)
    stamps = Stamps()

    def one_step(i: int, rec=None):
        ids = ids_base + i * 1_000_003  # a new prefix each step: a full store
        sp = stamps.span(stream) if rec is not None else None
        pc.store(ids, T, hidden, states, kv=(cache, pages))
        if rec is not None:
            rec.append(("store", sp.end(stream)))
            sp = stamps.span(stream)
        hit = pc.lookup_kv(ids, dev, cache)
        if rec is not None:
            rec.append(("restore", sp.end(stream)))
            sp = stamps.span(stream)
        hit2 = pc.lookup(ids, dev)
        if rec is not None:
            rec.append(("restore_dense", sp.end(stream)))
        assert hit is not None and hit2 is not None and len(hit[3]) == n_pages
        cache.free_pages(hit[3])

    log(f"entry: {entry_bytes / 2**20:.1f} MiB (hidden + states {dense_bytes / 2**20:.1f}, "
        f"KV {kv_bytes / 2**20:.1f})")
    for i in range(warmup):
        one_step(i)
    torch.cuda.synchronize()
    recs = [[] for _ in range(steps)]
    t0 = time.perf_counter()
    for j in range(steps):
        one_step(warmup + j, recs[j])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    pc.sync()
    cache.check_errors()
    # the last restore equals the source (bit-exact)
    ids = ids_base + (warmup + steps - 1) * 1_000_003
    hit = pc.lookup_kv(ids, dev, cache)
    torch.cuda.synchronize()
    pc.sync()
    exact = (torch.equal(hit[1], hidden) and all(torch.equal(a, b) for a, b in zip(hit[2], states))
             and torch.equal(cache.cache[:, :, hit[3]], cache.cache[:, :, pages]))
    cache.free_pages(hit[3])
    # the link's own DMA rate on the same box: a contiguous pinned copy each way
    host = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    devb = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dma = {}
    for name, fn in (("d2h", lambda: host.copy_(devb, non_blocking=True)),
                     ("h2d", lambda: devb.copy_(host, non_blocking=True))):
        fn()
        torch.cuda.synchronize()
        sp = stamps.span(stream)
        for _ in range(5):
            fn()
        sp.end(stream)
        torch.cuda.synchronize()
        dma[name] = 5 * host.numel() / (sp.ms() / 1e3) / 1e9
    st_ms, rs_ms, rd_ms = (_timed(recs, "store"), _timed(recs, "restore"),
                           _timed(recs, "restore_dense"))
    value = 2 * entry_bytes / ((st_ms + rs_ms) / 1e3) / 1e9
    res = {
        "metric": ("host-tier store + restore GB/s across the host link for a 32K-token "
                   "prefix-cache entry (hidden, 45 GDN states, 15 layers of KV pages)"),
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(elapsed / steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 + fp32 (bytes moved as is)",
        "data": "synthetic (seeded ~N(0,1) hidden, states and KV; shuffled pool pages)",
        "config": {"workload": (f"prefix-cache host tier, one rank: store then restore of a "
                                f"{T}-token prefix entry: hidden [{T}, {hidden_size}] bf16, "
                                f"{n_gdn} GDN states [1,8,128,128] fp32, KV of {LAYERS} layers "
                                f"x {n_pages} pages (1 KV head x 256, bf16) restored into fresh "
                                f"pages; pinned arena"),
                   "entry_bytes": entry_bytes},
        "store_ms": round(st_ms, 3), "restore_ms": round(rs_ms, 3),
        "store_GBps": round(entry_bytes / st_ms / 1e6, 2),
        "restore_GBps": round(entry_bytes / rs_ms / 1e6, 2),
        "restore_hidden_and_states_ms": round(rd_ms, 3),
        "restore_hidden_and_states_note": ("the reference's entry content alone; its docstring "
                                           "claims ~25 ms per 32K prefix "
                                           "(muserve/model/prefix_cache.py:4)"),
        "restored_bit_exact": bool(exact),
        "dma_ceiling_GBps": {k: round(v, 2) for k, v in dma.items()},
        "roofline": {
            "bound": "host link",
            "kernel": ("mkv_pack_blocks / mkv_unpack_blocks (KV, zero-copy into pinned memory) "
                       "+ hipMemcpyAsync (hidden, states)"),
            "achieved": round(value, 2), "peak": HOST_LINK_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HOST_LINK_PEAK_GBS, 4), "traffic": None,
            "frac_of_measured_dma": round(value / (0.5 * (dma["d2h"] + dma["h2d"])), 4),
        },
    }
    if with_cpu:
        # the reference's own path: tensor.cpu() into pageable memory, then
        # .to(device, non_blocking=True) from it (prefix_cache.py:36-44), for
        # the content it stores (hidden + states)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        stored = [t.cpu() for t in [hidden] + states]
        t2 = time.perf_counter()
        back = [t.to(dev, non_blocking=True) for t in stored]
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        assert all(torch.equal(a, b) for a, b in zip(back, [hidden] + states))
        res["cpu_baseline"] = {
            "value": round(2 * dense_bytes / (t3 - t1) / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"the reference's store / restore of hidden + {n_gdn} states "
                       f"({dense_bytes / 2**20:.0f} MiB; pageable tensor.cpu(), then "
                       f".to(device)): {1e3 * (t2 - t1):.1f} ms + {1e3 * (t3 - t2):.1f} ms"),
        }
    return res


def run_calibration(reps: int = 5, nbytes: int = 1 << 30) -> dict:
    """A plain device copy of known size (one 1 GiB state-pool entry through
    mkv_state_gather): the reference point for scaling rocprof's FETCH_SIZE and
    WRITE_SIZE counters to bytes."""
    from muserve_amd import _lib

    dev = torch.device("cuda:0")
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    slots = torch.zeros(1, dtype=torch.int32, device=dev)
    err = _lib.DeviceErrors(dev)
    for _ in range(reps):
        _lib.call("mkv_state_gather", src.data_ptr(), nbytes, dst.data_ptr(), None, 0, None, 1,
                  slots.data_ptr(), 1, err.ptr(), _lib.stream_of(dev))
    torch.cuda.synchronize()
    err.check("calibration copy")
    assert torch.equal(src, dst)
    return {"calibration": "state_move_kernel<true> copy", "bytes_read": nbytes,
            "bytes_written": nbytes, "launches": reps}


def run_ceilings(steps: int, warmup: int, with_cpu: bool) -> dict:
    """Access-pattern ceilings: the probe kernels (mkv_probe_*) and torch's own
    copies move the bytes of the product kernels in the same placement and do
    nothing else; each is timed with HIP events over `steps` launches after
    `warmup`. The product kernels' own rates come from their workloads."""
    from muserve_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    sp = _lib.stream_of(dev)
    sink = torch.zeros(16384, dtype=torch.uint8, device=dev)
    out: list[dict] = []

    def timed(fn) -> float:  # mean us per call
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    def record(probe: str, pattern: str, nbytes: int, us: float, **extra) -> None:
        gbs = nbytes / us / 1e3
        out.append({"probe": probe, "pattern": pattern, "bytes_per_launch": int(nbytes),
                    "mean_launch_us": round(us, 2), "GBps": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4), **extra})
        log(f"{probe} [{pattern}]: {us:.1f} us, {gbs:.0f} GB/s")

    # decode attention and the gather's data tiles: the K and V planes of one
    # layer's pages of the 256 lognormal sequences, every page once, shuffled
    ctx = context_lengths()
    npg = int(np.sum(-(-ctx // 16)))
    perm = torch.randperm(npg, generator=torch.Generator().manual_seed(SEED))
    perm_d = perm.to(torch.int32).to(dev)
    for pb, pool in ((8192, "bf16"), (4096, "fp8")):
        kp = torch.empty(npg * pb, dtype=torch.uint8, device=dev)
        vp = torch.empty_like(kp)
        for walk, nt, shape in ((0, 1, "a workgroup per page, non-temporal loads"),
                                (1, 0, "a wave per page, resident grid, cached loads"),
                                (1, 1, "a wave per page, resident grid, non-temporal loads")):
            us = timed(lambda: _lib.call("mkv_probe_read_pages", kp.data_ptr(), vp.data_ptr(), pb,
                                         npg, perm_d.data_ptr(), npg, walk, nt, sink.data_ptr(), sp))
            record("mkv_probe_read_pages", f"{pool} pages ({pb} B K + {pb} B V), {npg} pages "
                   f"shuffled, loads only: {shape}", 2 * npg * pb, us)
        if pb == 8192:
            # torch's copies of the same bytes (read and written): random pages
            # gathered (index_select) and a contiguous copy
            kp2, vp2 = kp.view(npg, pb), vp.view(npg, pb)
            ko, vo = torch.empty_like(kp2), torch.empty_like(vp2)
            idx = perm.to(dev)

            def isel():
                torch.index_select(kp2, 0, idx, out=ko)
                torch.index_select(vp2, 0, idx, out=vo)

            record("torch.index_select", f"{npg} shuffled 8 KiB pages of K and V gathered "
                   "to contiguous rows", 4 * npg * pb, timed(isel))

            def cpy():
                ko.copy_(kp2)
                vo.copy_(vp2)

            record("torch.Tensor.copy_", f"the same {2 * npg * pb} bytes, contiguous",
                   4 * npg * pb, timed(cpy))
            del ko, vo
        del kp, vp
        torch.cuda.empty_cache()

    # fp8 append: a 2048-token chunk of 32 requests (4096 pages) into a
    # 262,160-page pool, 15 layers per launch and one, shuffled or
    # consecutive pages; bf16 rows in (8 KiB a page), 4 KiB page rows out
    R, CHUNK, CTX = 32, 2048, 131072
    dpages = R * CTX // 16 + 16
    cpages = R * CHUNK // 16
    planes = 2 * LAYERS
    src = torch.empty(planes, cpages * 8192, dtype=torch.uint8, device=dev)
    dst = torch.empty(planes, dpages * 4096, dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(SEED)
    placements = {"shuffled": torch.randperm(dpages, generator=g)[:cpages],
                  "consecutive": torch.arange(cpages) + dpages // 2}
    for name, pg in placements.items():
        assert int(pg.min()) >= 0 and int(pg.max()) < dpages
        pg_d = pg.to(torch.int32).to(dev)
        for per_launch in (planes, 2):
            def scat():
                for i in range(0, planes, per_launch):
                    _lib.call("mkv_probe_scatter_pages", src[i].data_ptr(), src.stride(0),
                              dst[i].data_ptr(), dst.stride(0), dpages, pg_d.data_ptr(), cpages,
                              per_launch, sp)

            us = timed(scat)
            record("mkv_probe_scatter_pages", f"{cpages} pages {name}, {per_launch // 2} "
                   f"layer(s) per launch", planes * cpages * (8192 + 4096), us,
                   us_per_layer=round(us / LAYERS, 2))
    del src, dst
    torch.cuda.empty_cache()

    # the padded gather's zero tiles: a 6 GiB streaming fill
    fill = torch.empty(6 << 30, dtype=torch.uint8, device=dev)
    record("mkv_probe_fill", "16-byte device-scope non-temporal stores, 6 GiB",
           fill.numel(), timed(lambda: _lib.call("mkv_probe_fill", fill.data_ptr(),
                                                 fill.numel(), sp)))
    del fill
    torch.cuda.empty_cache()
    return {"metric": "access-pattern ceilings (probe kernels)", "value": None, "unit": "GB/s",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "higher_is_better": True,
            "dtype": "u8", "data": "synthetic (uninitialised planes, seeded page orders)",
            "config": {"workload": "ceilings"}, "probes": out}


def _summary(r: dict, keep: tuple[str, ...]) -> dict:
    """A secondary configuration's result, compacted for the headline line:
    its metric and value, the named extra keys, and per kernel the
    algorithmic bytes per launch, the event-timed mean launch and the
    fraction of the HBM roofline."""
    def kern(k: dict) -> dict:
        return {key: k[key] for key in ("kernel", "bound", "algorithmic_bytes_per_launch",
                                         "mean_launch_us", "achieved", "frac",
                                         "traffic_to_algorithmic", "us_per_request", "launch_ms",
                                         "GB_hashed_per_s") if key in k}
    out = {"workload": r["config"]["workload"], "metric": r["metric"], "value": r["value"],
           "unit": r["unit"], "ms_per_step": r["ms_per_step"]}
    out.update({k: r[k] for k in keep if k in r})
    roof = r["roofline"]
    out["kernels"] = [kern(k) for k in (roof["kernels"] if "kernels" in roof else [roof])]
    if "mall_cold" in r:
        out["mall_cold"] = {"pct_of_hbm_peak": r["mall_cold"]["pct_of_hbm_peak"],
                            "kernels": [kern(k) for k in r["mall_cold"]["kernels"]]}
    return out


def run_secondary() -> dict:
    """The other configurations, after the headline (each on a fresh pool,
    with its default sizes): fp8 chunked prefill, GDN state slots in model
    order (and MALL-cold), the prefix cache, paged decode attention over
    bf16 and fp8 pools at the headline's shape, and the continuous-batching
    serving step driven by the scheduler's step plan."""
    out = {}
    for name, fn, steps, warmup, keep in (
            ("fp8_prefill", run_fp8_prefill, 12, 3, ("pct_of_hbm_peak", "appended_tokens_per_s")),
            ("gdn_state", run_gdn_state, 50, 5, ("pct_of_hbm_peak", "state_move_ms_per_step")),
            ("prefix", run_prefix, 5, 1, ("requests_per_s", "phase_ms", "evictions",
                                          "page_hit_rate", "cow_copies")),
            # 50 warm-up steps: the fp8 attention's launches shorten over a
            # run's first 15-20 steps (145-150 us, then 134-140 us a launch)
            ("decode_attn", run_decode_attn, 200, 50, ("pct_of_hbm_peak", "tokens_per_s")),
            ("decode_attn_fp8", lambda st, wu, cpu: run_decode_attn(st, wu, cpu, fp8=True), 200,
             50, ("pct_of_hbm_peak", "tokens_per_s")),
            ("sched", run_sched, 500, 300, ("tokens_per_s", "attn_us_per_layer",
                                            "prefill_attn_us_per_layer"))):
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        log(f"secondary: {name}")
        out[name] = _summary(fn(steps, warmup, False), keep)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--calibrate", action="store_true",
                    help="run only a 1 GiB plain copy (for rocprof counter scaling)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="default workload: skip the other configurations after the headline")
    ap.add_argument("--serial-prefill", action="store_true",
                    help="sched workloads: prefill attention on the main stream, after the "
                         "decode attention (default: beside it on a second stream)")
    ap.add_argument("--placement", choices=("shuffled", "contiguous"), default="shuffled",
                    help="fp8_prefill: pool pages from a shuffled free list (default) or "
                         "consecutive pages per request (to measure what the scatter costs)")
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "fp8_prefill", "gdn_state", "plumbing", "prefix",
                             "decode_attn", "decode_attn_fp8", "offload", "gdn_decode",
                             "sched", "sched_fp8", "sched_hybrid", "sched_prefix",
                             "prefill_attn", "ceilings"],
                    help="decode (default, the headline metric) or another configuration")
    args = ap.parse_args()
    global PLACEMENT
    PLACEMENT = args.placement
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this path has no cross-GPU traffic "
              "(each tensor-parallel rank owns its own pool); run with --gpus 1",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    if args.calibrate:
        print(json.dumps(run_calibration()), flush=True)
        return 0
    runner = {"decode": run_decode, "fp8_prefill": run_fp8_prefill, "gdn_state": run_gdn_state,
              "plumbing": run_plumbing, "prefix": run_prefix,
              "decode_attn": run_decode_attn,
              "decode_attn_fp8": lambda *a: run_decode_attn(*a, fp8=True),
              "offload": run_offload,
              "gdn_decode": lambda *a: run_gdn_state(*a, fused_conv=True),
              "sched": lambda *a: run_sched(*a, serial_prefill=args.serial_prefill),
              "sched_fp8": lambda *a: run_sched(*a, fp8=True),
              "sched_hybrid": lambda *a: run_sched(*a, hybrid=True,
                                                   serial_prefill=args.serial_prefill),
              "sched_prefix": lambda *a: run_sched(*a, prefix=True,
                                                   serial_prefill=args.serial_prefill),
              "prefill_attn": run_prefill_attn, "ceilings": run_ceilings}[args.workload]
    steps, warmup = args.steps, args.warmup
    if args.workload == "fp8_prefill" and steps == 1000:
        steps, warmup = 12, 3  # 15 chunks of 2048 fit before the 8192-token window
    if args.workload == "prefix" and steps == 1000:
        steps, warmup = 5, 1  # a step is the whole 4096-request trace
    if args.workload == "offload" and steps == 1000:
        steps, warmup = 10, 2  # a step moves ~1.5 GB across the host link
    if args.workload == "prefill_attn" and (steps, warmup) == (1000, 20):
        steps, warmup = 20, 3
    if args.workload == "ceilings" and (steps, warmup) == (1000, 20):
        steps, warmup = 20, 3
    if args.workload.startswith("sched") and (steps, warmup) == (1000, 20):
        steps, warmup = 500, 300  # the warmup fills the 256-request batch
    # a garbage-collector pass in the timed loop stalls the host for tens of
    # ms, the stream drains and the event span around the launch absorbs the
    # pause: collect once, freeze what setup allocated and keep the collector
    # off (the bench frees its buffers by reference counting)
    gc.collect()
    gc.freeze()
    gc.disable()
    res = runner(steps, warmup, not args.no_cpu_baseline)
    if args.workload == "decode" and not args.no_secondary:
        res["secondary"] = run_secondary()
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
