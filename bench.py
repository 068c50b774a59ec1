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
``cpu_baseline`` times the CPU oracle's gather on one layer of one step.
"""
from __future__ import annotations

import argparse
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


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def context_lengths(seed: int = SEED) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.clip(np.round(rng.lognormal(np.log(4096.0), 1.0, B)), 1, 32768).astype(np.int64)


def step_bytes(lens: np.ndarray) -> tuple[float, float, float]:
    """(all algorithmic bytes of one step, of one gather launch, useful bytes of
    one step without padding writes) for post-append lengths ``lens``."""
    lpad = int(-(-int(lens.max()) // 16) * 16)
    nblk = -(-lens // 16)
    gather = 2 * ROW * lens.sum() + 2 * ROW * B * lpad + 4 * nblk.sum() + 4 * B
    append = 2 * B * ROW + 2 * B * ROW + 8 * B
    useful = 2 * B * ROW + 2 * B * ROW + 8 * B + 4 * ROW * lens.sum() + 4 * nblk.sum() + 4 * B
    return float(LAYERS * (gather + append)), float(gather), float(LAYERS * useful)


def cpu_baseline(cache, bt, lens_now: np.ndarray, gpu_out) -> dict:
    """The oracle's gather (torch-CPU index_select per sequence) on the last
    layer of the current step, timed on the host; also checks the GPU result
    of that layer (the last one the timed loop gathered) against it."""
    from oracle import paged as ref

    threads = torch.get_num_threads()
    lpad = int(gpu_out[0].shape[1])
    kplane = cache.cache[LAYERS - 1, 0].cpu()
    vplane = cache.cache[LAYERS - 1, 1].cpu()
    bt_cpu = bt.tables.cpu()
    sl = torch.from_numpy(lens_now.astype(np.int32))
    t0 = time.perf_counter()
    k_ref = ref.gather_padded(kplane, bt_cpu, sl, lpad)
    v_ref = ref.gather_padded(vplane, bt_cpu, sl, lpad)
    dt = time.perf_counter() - t0
    _, gbytes, _ = step_bytes(lens_now)
    same = bool(torch.equal(gpu_out[0].cpu().view(torch.int16), k_ref.view(torch.int16)) and
                torch.equal(gpu_out[1].cpu().view(torch.int16), v_ref.view(torch.int16)))
    return {
        "value": round(gbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle gather (torch-CPU index_select, {threads} threads) of one layer's K, V "
                   f"of one decode step at batch {B}, Lpad {lpad}: {dt:.2f} s"),
        "seconds": round(dt, 3),
        "cpu_model": _cpu_model(),
        "gpu_matches_cpu_on_sampled_layer": same,
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
    total_steps = warmup + steps
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

    def one_step(i: int, events=None):
        slots = bt.decode_step()
        lpad = bt.padded_len()
        kout = kbuf[:B * lpad * HEAD_DIM].view(B, lpad, 1, HEAD_DIM)
        vout = vbuf[:B * lpad * HEAD_DIM].view(B, lpad, 1, HEAD_DIM)
        for l in range(LAYERS):
            cache.append(slots, kin[i, l], vin[i, l], layer=l)
            if events is not None:
                events[l][0].record(stream)
            cache.gather(l, bt.tables, bt.seq_lens, out_len=lpad, out=(kout, vout))
            if events is not None:
                events[l][1].record(stream)
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
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(LAYERS)]
          for _ in range(steps)]
    log(f"timing {steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for j in range(steps):
        out = one_step(warmup + j, ev[j])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    cache.check_errors()
    gather_ms = [e[0].elapsed_time(e[1]) for step in ev for e in step]
    mean_gather_s = float(np.mean(gather_ms)) / 1e3
    mean_gather_bytes = gather_bytes / steps
    lens_now = bt._lens.copy()

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
            "traffic": traffic,
            "traffic_to_algorithmic": ratio,
            "traffic_source": ("rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 (scales from a 1 GiB copy), "
                               "profiles/gather_decode_b256_hbm_counters.md"),
            "mean_launch_us": round(mean_gather_s * 1e6, 2),
            "algorithmic_bytes_per_launch": round(mean_gather_bytes),
        },
    }
    if with_cpu:
        log("cpu baseline (one layer of one step)")
        res["cpu_baseline"] = cpu_baseline(cache, bt, lens_now, out)
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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--calibrate", action="store_true",
                    help="run only a 1 GiB plain copy (for rocprof counter scaling)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
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
    res = run_decode(args.steps, args.warmup, not args.no_cpu_baseline)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
