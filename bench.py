"""Benchmark of the KV-cache hot path on one MI355X.

A step is one engine decode step's worth of hot-path work for the GQA decode
workload (64 rows, ctx U[128, 2048], 32/8 heads, D=128, bf16, block 16, pool
1.25x shuffled): for each of 32 layers, the 64-token KV append
(kvhot_reshape_and_cache) and the split-K paged decode attention
(kvhot_paged_attention) over that layer's pool.  Each layer has its own
~348 MB pool (11 GB in all), so a layer's K/V is never still resident in the
256 MB Infinity Cache when it is read again.  The pool is the drop-in's
documented one, allocate_kv_cache()'s default: the reference's
[L, 2, N, 16, Hkv, D] shape and indexing with each block stored as
[Hkv, 2, 16, D] (kv-interleaved: each kv head's 16 K rows, then its 16 V
rows); `reference_layout` and `head_major_layout` are the same calls on the
reference's token-major [16, Hkv, D] blocks and on head-major [Hkv, 16, D]
blocks with the K and V pools apart (--layout makes either the headline).

value = algorithmic bytes moved per step (K/V read + Q in + O out + block
table + LSE out, plus the append's K/V read+write and slots) / step time, in
GB/s (1e9).  roofline = one attention call alone (the decode launch, plus a
merge launch when the plan cuts a row across work-groups): its algorithmic
bytes over its average duration, timed with HIP events on the launch stream
across replays of one recorded HIP graph of 32 back-to-back calls (device
time per launch; the eager per-call time, host dispatch included, is
reported beside it); `traffic` = the HBM bytes rocprofv3's FETCH_SIZE and
WRITE_SIZE counters read for the same call, scaled by what they read for a
copy of known size, as recorded in profiles/ (null when that file is
absent).  deterministic = the same calls with deterministic=True
(KVHOT_DETERMINISTIC: bitwise-repeatable results).

Other legs, each one attention (or append) call timed the same way over
its own layer pools:
* append_large: the mixed workload's 4,152-token append (8 x 512-token
  chunks + 56 decode tokens), GB/s of K/V read + written against 8 TB/s;
* prefix: the prefix-sharing workload (256 decode rows sharing 64 blocks,
  private tails U[64, 512]), GB/s on the unique K/V bytes (the shared prefix
  once) and on the logical ones (every row's keys);
* long_context: the long-context workload (16 rows x 32,768 tokens over a
  40 GB pool, 512-token split-K partitions), GB/s; `planner_split` the same
  call with the planner choosing the split (the drop-in's default);
* prefill: the chunked-prefill rows of the mixed workload (8 x 512-token
  chunks on contexts U[0, 4096]): one attention call over them, FLOPs
  counted over visible (query, key) pairs only, against the 2.5 PFLOP/s
  dense bf16 MFMA peak; the whole mixed batch and its 56 decode rows alone
  are timed alongside;
* copy: kvhot_copy_blocks over the prefix-sharing workload's 256
  copy-on-write pairs on a 32-layer pool (1 GiB read and written per
  launch);
* engine: output tokens/s of greedy decode steps of a random-weight
  Llama-3.1-8B-shaped model (32 layers, hidden 4096, 32/8 heads, D=128,
  vocab 128256, bf16) whose attention is paged|hip over a paged pool, 64
  sequences with contexts U[128, 2048] (synthetic context K/V, the whole
  model every step; the step recorded once in a HIP graph and replayed, the
  eager step beside it), with the same model on the host CPU (the
  reference's eager attention restated in oracle/eager.py; 1, 2 and 4
  layers, the per-layer time fitted) as its baseline;
* cpu_baseline: the reference's eager PyTorch path (restated in
  oracle/eager.py) on this host's cores, on one layer of the same batch;
* host_step: host time per engine step of the metadata and of the attention
  launch list.
Every per-launch figure is a median over --kernel-reps HIP-event timings.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 2]
       python bench.py --headline-only   # the step and its attention call only
                                         # (counter runs)
       python bench.py --copy-probe      # kvhot_copy_blocks of 256 MiB each way
                                         # (counter calibration)
       python bench.py --prefill-only    # the prefill measurement alone
       python bench.py --legs-only       # the append_large, prefix and long_context legs alone
       python bench.py --copy-only       # the copy-on-write block copy alone
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILES = {
    "reference": os.path.join(ROOT, "profiles", "attention_decode_gqa64_traffic.md"),
    "head-major": os.path.join(ROOT, "profiles", "attention_decode_gqa64_headmajor_traffic.md"),
    "kv-interleaved": os.path.join(ROOT, "profiles", "attention_decode_gqa64_kvinterleaved_traffic.md"),
}
LAYOUT_NAMES = {"kv-interleaved": "kv-interleaved blocks [Hkv, 2, 16, D]: each kv head's K rows, then its V rows "
                                  "(allocate_kv_cache's default)",
                "head-major": "head-major blocks [Hkv, 16, D], the K and V pools apart",
                "reference": "the reference's token-major blocks [16, Hkv, D]"}
# allocate_kv_cache's name of each --layout, and the line's key for its figures
# when it is not the headline
POOL_LAYOUT = {"kv-interleaved": "kv-interleaved", "head-major": "head-major", "reference": "token-major"}
OTHER_KEYS = {"reference": "reference_layout", "head-major": "head_major_layout",
              "kv-interleaved": "kv_interleaved_layout"}
DEFAULT_POOL = "kv-interleaved"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", type=int, default=2, choices=[2, 3, 4, 5])
    ap.add_argument("--layout", choices=sorted(LAYOUT_NAMES), default=DEFAULT_POOL,
                    help="how the pool stores a block: kv-interleaved [Hkv, 2, 16, D] (allocate_kv_cache's "
                         "default), head-major [Hkv, 16, D] or the reference's token-major [16, Hkv, D]")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--partition-tokens", type=int, default=0)
    ap.add_argument("--kernel-reps", type=int, default=20,
                    help="timed passes over all layers for the per-launch figures (their median is reported)")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the step and its attention call on the headline layout (for counter runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill MFMA measurement")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill measurement (for counter runs); prints its JSON object")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the append_large, prefix and long_context legs")
    ap.add_argument("--legs-only", action="store_true",
                    help="only the append_large, prefix and long_context legs; prints their JSON objects")
    ap.add_argument("--no-engine", action="store_true", help="skip the engine tokens/s measurement")
    ap.add_argument("--no-copy", action="store_true", help="skip the copy-on-write block copy measurement")
    ap.add_argument("--copy-only", action="store_true",
                    help="only the copy-on-write block copy measurement; prints its JSON object")
    ap.add_argument("--engine-only", action="store_true", help="only the engine measurement")
    ap.add_argument("--engine-steps", type=int, default=16)
    ap.add_argument("--engine-cpu-layers", type=str, default="1,2,4",
                    help="layer counts of the CPU engine baseline (the per-layer time is fitted over them)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="budget for the CPU baseline sample")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run kvhot_copy_blocks over 256 MiB each way, 5 times (counter calibration)")
    return ap.parse_args()


def launch_list_desc(meta, w):
    """The launches of one attention call, from the unit counts of its launch
    list (kvhot_paged_attention_schedule)."""
    import torch

    plans = [p for p in meta.get("_schedules", {}).values() if p is not None]
    if not plans:
        return "one attention call on the padded grid (no launch list)"
    _, n_dec, n_pre, n_mrg, _, n_pfx = plans[0]
    tt = "BF16" if w.dtype == torch.bfloat16 else "F16"
    parts = []
    if n_pfx:
        parts.append(f"attn_prefill_kernel<{tt},{w.head_dim}> x {n_pfx} shared-prefix units")
    if n_pre > n_pfx:
        parts.append(f"attn_prefill_kernel<{tt},{w.head_dim}> x {n_pre - n_pfx} units")
    if n_dec:
        # one range per wave, or up to four per wave with fixed partitions
        parts.append(f"attn_decode_kernel<{tt},{w.head_dim}> x {n_dec} ranges")
    if n_mrg:
        parts.append(f"attn_merge_kernel<{tt},{w.head_dim}> x {n_mrg} units")
    return "one attention call: " + " + ".join(parts)


def median_pass_us(body, reps):
    """Median device time of `reps` runs of body(), each bracketed by HIP
    events on the current stream, in microseconds."""
    import torch

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    for a, b in ev:
        a.record()
        body()
        b.record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) * 1e3 for a, b in ev)


def host_threads():
    """Host threads for the CPU baselines: every CPU this process may run on,
    within OMP_NUM_THREADS when that is set (a shared host's share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model():
    """The host CPU's model string (/proc/cpuinfo), or the platform's."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def recorded_traffic(workload: int, layout: str):
    """HBM bytes per attention call recorded from the rocprofv3 counter runs
    (a `traffic_bytes_per_call: N` line of the layout's file under
    profiles/), for workload 2."""
    path = TRAFFIC_FILES.get(layout)
    if workload != 2 or path is None or not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.strip().startswith("traffic_bytes_per_call:"):
                return int(line.split(":", 1)[1].strip())
    return None


def per_call_us(body, calls, reps, dev):
    """(graph, eager) per-call device time of body(), which makes `calls`
    back-to-back calls: medians over `reps` passes, run eagerly (host
    dispatch included) and as replays of one recorded HIP graph of the pass
    (device time per call: what a kernel trace's average is compared with)."""
    import torch

    torch.cuda.synchronize()
    eager = median_pass_us(body, reps) / calls
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        body()  # every lazy set-up done before the recording
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        body()
    graph.replay()
    torch.cuda.synchronize()
    us = median_pass_us(graph.replay, reps) / calls
    del graph
    return us, eager


def copy_probe():
    """kvhot_copy_blocks of 4096 block pairs (K and V, 32 KiB each): 256 MiB
    read and 256 MiB written per launch, the known-size copy the counter
    readings are scaled by."""
    import torch

    sea = importlib.import_module("serving-engine_amd")
    dev = torch.device("cuda:0")
    kv = torch.zeros((1, 2, 8192, 16, 8, 128), dtype=torch.bfloat16, device=dev)
    cache = sea._PagedKVCache(kv)
    src = torch.arange(0, 4096, dtype=torch.int64)
    dst = torch.arange(4096, 8192, dtype=torch.int64)
    for _ in range(5):
        cache.copy_blocks(src, dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe": "kvhot_copy_blocks", "pairs": 4096, "read_bytes": 2 * 4096 * 32768,
                      "write_bytes": 2 * 4096 * 32768, "launches": 5}), flush=True)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path", file=sys.stderr)
        sys.exit(2)

    if args.copy_probe:
        copy_probe()
        return
    if args.engine_only:
        import torch

        torch.cuda.set_device(0)
        print(json.dumps({"engine": engine_measure(torch.device("cuda:0"), steps=args.engine_steps,
                                                   cpu_layers=[] if args.no_cpu_baseline else cpu_layer_counts(args))}),
              flush=True)
        return
    if args.copy_only:
        import torch

        torch.cuda.set_device(0)
        sea = importlib.import_module("serving-engine_amd")
        wl = importlib.import_module("serving-engine_amd.workloads")
        print(json.dumps({"copy": copy_measure(sea, wl, torch.device("cuda:0"), reps=max(1, args.kernel_reps))}),
              flush=True)
        return
    if args.legs_only:
        import torch

        torch.cuda.set_device(0)
        sea = importlib.import_module("serving-engine_amd")
        wl = importlib.import_module("serving-engine_amd.workloads")
        dev = torch.device("cuda:0")
        reps = max(1, args.kernel_reps)
        print(json.dumps({"append_large": append_leg(sea, wl, dev, reps),
                          "prefix": attention_leg(sea, wl, dev, 4, layers=16, reps=reps),
                          "long_context": attention_leg(sea, wl, dev, 5, layers=1, reps=max(3, reps // 2), calls=8)}),
              flush=True)
        return
    if args.prefill_only:
        import torch

        torch.cuda.set_device(0)
        sea = importlib.import_module("serving-engine_amd")
        wl = importlib.import_module("serving-engine_amd.workloads")
        print(json.dumps({"prefill": prefill_measure(sea, wl, torch.device("cuda:0"),
                                                     reps=max(1, args.kernel_reps))}), flush=True)
        return

    import torch

    sea = importlib.import_module("serving-engine_amd")
    wl = importlib.import_module("serving-engine_amd.workloads")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    w = wl.make_workload(args.workload)
    layers = args.layers if args.workload != 5 else 1  # the 40 GB pool is one layer's
    t = wl.make_tensors(w, dev, num_layers=layers, layout=POOL_LAYOUT[args.layout])
    cache = sea._PagedKVCache(t.kv_cache)
    meta = sea.build_paged_batch_metadata(w.scheduler_output(), device=dev)
    slots = meta["slot_mapping"]
    scale = 1.0 / math.sqrt(w.head_dim)
    pt = args.partition_tokens or w.partition_tokens or None
    blocks = [cache.blocks(i) for i in range(layers)]

    def attention(i, bl=blocks, deterministic=False):
        return sea.paged_flash_attention(t.q, bl[i][0], bl[i][1], meta, w.num_q_heads,
                                         w.num_kv_heads, scale, partition_tokens=pt, deterministic=deterministic)

    def step():
        for i in range(layers):
            cache.write(t.new_k, t.new_v, i, slots)
            attention(i)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps

    attn_bytes = w.decode_algorithmic_bytes()
    append_bytes = w.append_bytes()
    step_bytes = layers * (attn_bytes + append_bytes)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # Attention and append alone: back-to-back launches over the layers.
    reps = max(1, args.kernel_reps)
    attn_us, attn_eager_us = per_call_us(lambda: [attention(i) for i in range(layers)], layers, reps, dev)
    attn_gbs = attn_bytes / (attn_us * 1e-6) / 1e9
    append_us, append_eager_us = per_call_us(
        lambda: [cache.write(t.new_k, t.new_v, i, slots) for i in range(layers)], layers, reps, dev)

    others, deterministic = {}, None
    if not args.headline_only:
        # The same calls on a copy of the pool in each other block layout
        # (same shape, values and results), and with deterministic=True.
        for other_layout in sorted(LAYOUT_NAMES):
            if other_layout == args.layout:
                continue
            kv2 = sea.allocate_kv_cache(layers, w.num_blocks, w.num_kv_heads, w.head_dim, dtype=w.dtype,
                                        device=dev, layout=POOL_LAYOUT[other_layout])
            kv2.copy_(t.kv_cache)
            blocks2 = [(kv2[i, 0], kv2[i, 1]) for i in range(layers)]
            o_us, _ = per_call_us(lambda: [attention(i, blocks2) for i in range(layers)], layers, reps, dev)
            del kv2, blocks2
            torch.cuda.empty_cache()
            o_gbs = attn_bytes / (o_us * 1e-6) / 1e9
            others[OTHER_KEYS[other_layout]] = {
                "pool_layout": LAYOUT_NAMES[other_layout], "avg_launch_us": round(o_us, 3),
                "achieved": round(o_gbs, 2), "unit": "GB/s", "frac": round(o_gbs / HBM_PEAK_GBS, 4),
                "traffic": recorded_traffic(args.workload, other_layout)}
        d_us, _ = per_call_us(lambda: [attention(i, deterministic=True) for i in range(layers)], layers, reps, dev)
        d_gbs = attn_bytes / (d_us * 1e-6) / 1e9
        deterministic = {"flag": "KVHOT_DETERMINISTIC (paged_flash_attention(..., deterministic=True))",
                         "pool_layout": LAYOUT_NAMES[args.layout], "avg_launch_us": round(d_us, 3),
                         "achieved": round(d_gbs, 2), "unit": "GB/s", "frac": round(d_gbs / HBM_PEAK_GBS, 4),
                         "cost_vs_default": round(d_us / attn_us - 1.0, 4)}

    host_cost = None if args.headline_only else host_step_cost(sea, w, dev, pt)

    cpu = None
    if not args.no_cpu_baseline and not args.headline_only:
        cpu = cpu_baseline(w, t, layer=0, budget_s=args.cpu_seconds, attn_bytes=attn_bytes + append_bytes)

    desc = launch_list_desc(meta, w)
    del t, cache, blocks
    torch.cuda.empty_cache()

    legs = {}
    if not args.headline_only and not args.no_legs:
        legs["append_large"] = append_leg(sea, wl, dev, reps)
        legs["prefix"] = attention_leg(sea, wl, dev, 4, layers=16, reps=reps)
        legs["long_context"] = attention_leg(sea, wl, dev, 5, layers=1, reps=max(3, reps // 2), calls=8)
    prefill = None
    if not args.no_prefill and not args.headline_only:
        prefill = prefill_measure(sea, wl, dev, reps=reps)
    copy = None if args.no_copy or args.headline_only else copy_measure(sea, wl, dev, reps=reps)
    engine = None
    if not args.no_engine and not args.headline_only:
        engine = engine_measure(dev, steps=args.engine_steps,
                                cpu_layers=[] if args.no_cpu_baseline else cpu_layer_counts(args))

    line = {
        "metric": "decode paged-attn HBM GB/s (% of 8 TB/s); engine output tokens/sec",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == torch.bfloat16 else str(w.dtype).replace("torch.", ""),
        "data": "synthetic",
        "config": {
            "workload": w.name,
            "layers_per_step": layers,
            "rows": len(w.rows),
            "total_context_tokens": int(sum(x.k_len for x in w.rows)),
            "block_size": w.block_size,
            "pool_blocks_per_layer": w.num_blocks,
            "append_tokens": w.total_query,
            "partition_tokens": pt or "auto",
            "seed": w.seed,
            "pool_layout": LAYOUT_NAMES[args.layout],
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": desc,
            "achieved": round(attn_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": recorded_traffic(args.workload, args.layout),
            "algorithmic_bytes_per_launch": attn_bytes,
            "avg_launch_us": round(attn_us, 3),
            "avg_launch_us_timing": f"HIP events over replays of one recorded graph of the {layers} back-to-back calls",
            "eager_call_us": round(attn_eager_us, 3),
            "pool_layout": LAYOUT_NAMES[args.layout],
        },
        **others,
        "deterministic": deterministic,
        "append": {"avg_launch_us": round(append_us, 3), "eager_call_us": round(append_eager_us, 3),
                   "algorithmic_bytes": append_bytes,
                   "gbs": round(append_bytes / (append_us * 1e-6) / 1e9, 2)},
        "host_step": host_cost,
        "cpu_baseline": cpu,
    }
    line.update(legs)
    if copy is not None:
        line["copy"] = copy
    if prefill is not None:
        line["prefill"] = prefill
    if engine is not None:
        line["engine"] = engine
    print(json.dumps(line), flush=True)


def cpu_layer_counts(args):
    return [int(x) for x in args.engine_cpu_layers.split(",") if x.strip()]


def append_leg(sea, wl, dev, reps, layers=16):
    """The mixed workload's append (8 x 512-token chunks + 56 decode tokens:
    4,152 tokens x 8 kv heads x 128 x bf16 for K and V) into `layers` layer
    pools: per-call time, GB/s of K/V read + written (+ slots) against 8 TB/s."""
    import torch

    w = wl.make_workload(3)
    t = wl.make_tensors(w, dev, num_layers=layers, layout=POOL_LAYOUT[DEFAULT_POOL])
    cache = sea._PagedKVCache(t.kv_cache)
    slots = t.slot_mapping
    us, eager = per_call_us(lambda: [cache.write(t.new_k, t.new_v, i, slots) for i in range(layers)],
                            layers, reps, dev)
    nbytes = w.append_bytes()
    gbs = nbytes / (us * 1e-6) / 1e9
    del t, cache
    torch.cuda.empty_cache()
    return {"workload": w.name, "kernel": "reshape_and_cache_kernel", "tokens": w.total_query,
            "algorithmic_bytes": nbytes, "avg_launch_us": round(us, 3), "eager_call_us": round(eager, 3),
            "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "timing": f"HIP events over replays of one recorded graph of {layers} back-to-back appends "
                      f"(one layer pool each), median of {reps}"}


def attention_leg(sea, wl, dev, config, layers, reps, calls=None):
    """One attention call of workload `config` on the default pool layout: per-call
    time over `calls` back-to-back calls cycling through `layers` layer pools,
    GB/s of its algorithmic bytes (logical: every row's keys; unique: each
    physical K/V byte once) against 8 TB/s.  A workload with fixed split-K
    partitions (the long-context one's 512 tokens) is also timed with the
    planner choosing the split (`planner_split`: paged_flash_attention
    without partition_tokens)."""
    import torch

    w = wl.make_workload(config)
    t = wl.make_tensors(w, dev, num_layers=layers, layout=POOL_LAYOUT[DEFAULT_POOL])
    cache = sea._PagedKVCache(t.kv_cache)
    meta = sea.build_paged_batch_metadata(w.scheduler_output(), device=dev)
    blocks = [cache.blocks(i) for i in range(layers)]
    scale = 1.0 / math.sqrt(w.head_dim)
    pt = w.partition_tokens or None
    calls = calls or layers

    def body():
        for c in range(calls):
            kc, vc = blocks[c % layers]
            sea.paged_flash_attention(t.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads, scale, partition_tokens=pt)

    us, eager = per_call_us(body, calls, reps, dev)
    logical = w.decode_algorithmic_bytes()
    unique = w.decode_algorithmic_bytes(unique=True)
    desc = launch_list_desc(meta, w)
    planner = None
    if pt:
        meta2 = sea.build_paged_batch_metadata(w.scheduler_output(), device=dev)

        def body2():
            for c in range(calls):
                kc, vc = blocks[c % layers]
                sea.paged_flash_attention(t.q, kc, vc, meta2, w.num_q_heads, w.num_kv_heads, scale)

        us2, _ = per_call_us(body2, calls, reps, dev)
        planner = {"kernel": launch_list_desc(meta2, w), "avg_call_us": round(us2, 3),
                   "achieved": round(logical / (us2 * 1e-6) / 1e9, 2), "unit": "GB/s",
                   "frac": round(logical / (us2 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del t, cache, blocks
    torch.cuda.empty_cache()
    out = {"workload": w.name, "kernel": desc, "avg_call_us": round(us, 3), "eager_call_us": round(eager, 3),
           "algorithmic_bytes": logical, "achieved": round(logical / (us * 1e-6) / 1e9, 2), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(logical / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "pool_layout": LAYOUT_NAMES[DEFAULT_POOL],
           "timing": f"HIP events over replays of one recorded graph of {calls} back-to-back calls over "
                     f"{layers} layer pool(s), median of {reps}"}
    if unique != logical:
        out["unique_bytes"] = unique
        out["unique_achieved"] = round(unique / (us * 1e-6) / 1e9, 2)
        out["unique_frac"] = round(unique / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    if pt:
        out["partition_tokens"] = pt
        out["planner_split"] = planner
    return out


class _DecodeRow:
    """A decode request as the metadata builder reads it (duck-typed Request:
    total_len, block_table, phase, num_computed_tokens, request_id)."""

    def __init__(self, rid, total_len, table, phase):
        self.request_id = rid
        self.total_len = total_len
        self.num_computed_tokens = total_len - 1
        self.block_table = table
        self.phase = phase


def _llama_8b_config(num_layers):
    from transformers import LlamaConfig

    return LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=num_layers,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                       max_position_embeddings=131072, rms_norm_eps=1e-5, rope_theta=500000.0,
                       rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                     "high_freq_factor": 4.0, "original_max_position_embeddings": 8192},
                       tie_word_embeddings=False)


def _random_llama(cfg, device, attn_impl):
    """LlamaForCausalLM in bf16 on `device`, built on the meta device and
    materialised without the library's initialisation; every weight is
    filled by tiling one seeded N(0, 0.02) block of 2^20 values (a timing
    model: the values only need to be finite and of a realistic scale)."""
    import torch
    from transformers import LlamaForCausalLM

    cfg._attn_implementation = attn_impl
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("meta"):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model = model.to_empty(device=device)
    model.eval()
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    block = torch.empty(1 << 20, dtype=torch.float32, device=device).normal_(0.0, 0.02, generator=gen)
    block = block.to(torch.bfloat16)
    with torch.no_grad():
        for prm in model.parameters():
            flat = prm.view(-1)
            for o in range(0, flat.numel(), block.numel()):
                m = min(block.numel(), flat.numel() - o)
                flat[o:o + m].copy_(block[:m])
    # Buffers (the rotary frequencies) are computed, not initialised weights:
    # rebuild that module on the device.
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    with torch.device(device):
        model.model.rotary_emb = LlamaRotaryEmbedding(config=cfg)
    return model


def _decode_batch(steps, seed=1002):
    """Context lengths of the GQA decode workload (64 x U[128, 2048], same
    seed) and shuffled block tables with room for `steps` more tokens."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ctx = rng.integers(128, 2048, size=64, endpoint=True)
    need = [math.ceil((int(c) + steps) / 16) for c in ctx]
    n = math.ceil(1.25 * sum(need))
    perm = rng.permutation(n)
    tables, k = [], 0
    for nb in need:
        tables.append([int(b) for b in perm[k:k + nb]])
        k += nb
    return [int(c) for c in ctx], tables, n


def engine_measure(dev, steps=16, warmup=2, cpu_layers=(1, 2, 4)):
    """Greedy decode steps of the random-weight Llama-3.1-8B-shaped model on
    paged|hip attention: output tokens/s over `steps` timed steps (metadata,
    append, attention, the whole forward and argmax each step), run eagerly
    and then as replays of the step recorded in a HIP graph
    (DecodeStepGraph), continuing the same sequences."""
    import torch

    sea = importlib.import_module("serving-engine_amd")
    layers = 32
    cfg = _llama_8b_config(layers)
    model = _random_llama(cfg, dev, sea.register_attention())
    ctx, tables, n = _decode_batch(2 * (warmup + steps))
    kv = sea.allocate_kv_cache(layers, n, 8, 128, dtype=torch.bfloat16, device=dev)  # the default layout
    gen = torch.Generator(device=dev)
    gen.manual_seed(1002)
    for lyr in range(layers):  # synthetic context K/V, N(0, 1) / sqrt(128)
        kv[lyr].normal_(0.0, 1.0 / math.sqrt(128), generator=gen)
    cache = sea._PagedKVCache(kv)
    lens = list(ctx)
    tok = torch.zeros(len(lens), dtype=torch.int64, device=dev)

    def step():
        nonlocal tok
        so = sea.SchedulerOutput()
        for i, (ln, tb) in enumerate(zip(lens, tables)):
            so.scheduled_requests.append(_DecodeRow(f"s{i}", ln + 1, tb, sea.RequestPhase.NEEDS_DECODE))
        meta = sea.build_paged_batch_metadata(so, device=dev)
        with torch.no_grad():
            out = model(input_ids=tok.view(1, -1), position_ids=meta["positions"].view(1, -1), cache=cache,
                        write_index=meta["slot_mapping"], paged_metadata=meta, use_cache=False)
        tok = out.logits[0].argmax(-1)
        for i in range(len(lens)):
            lens[i] += 1

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_eager = e0.elapsed_time(e1) / steps

    # The same step recorded once and replayed (continuing the sequences).
    graph = sea.DecodeStepGraph(model, cache, len(lens), max(len(t) for t in tables), 32, 8, 128, dev)
    graph.tokens.copy_(tok)

    def gstep():
        graph.step([ln + 1 for ln in lens], tables)
        for i in range(len(lens)):
            lens[i] += 1

    for _ in range(warmup):
        gstep()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        gstep()
    e1.record()
    torch.cuda.synchronize()
    gwall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    res = {
        "model": "Llama-3.1-8B-shaped, random N(0,0.02) weights, bf16: 32 layers, hidden 4096, ffn 14336, "
                 "32/8 heads, D=128, vocab 128256",
        "attention": "paged|hip (kvhot_reshape_and_cache + kvhot_paged_attention per layer)",
        "batch": len(lens),
        "context": "64 x U[128, 2048] tokens at the first step (synthetic K/V), +1 per step",
        "steps": steps,
        "step": "recorded once in a HIP graph (DecodeStepGraph) and replayed: per step the host builds the "
                "metadata and the attention launch list, two pinned copies, one graph launch",
        "ms_per_step": round(ms, 3),
        "ms_per_step_per_layer": round(ms / layers, 4),
        "tokens_per_s": round(len(lens) / (ms * 1e-3), 1),
        "wall_tokens_per_s": round(len(lens) * steps / gwall, 1),
        "graph_recordings": graph.recordings,
        "eager": {"ms_per_step": round(ms_eager, 3), "tokens_per_s": round(len(lens) / (ms_eager * 1e-3), 1),
                  "wall_tokens_per_s": round(len(lens) * steps / wall, 1)},
    }
    del graph, model, kv, cache
    torch.cuda.empty_cache()
    if cpu_layers:
        res["cpu_baseline"] = engine_cpu_baseline(cpu_layers, ctx, tables, n)
    return res


def engine_cpu_baseline(layer_counts, ctx, tables, n, steps=5):
    """The same decode step on the host CPU with the reference's eager paged
    attention (restated in oracle/eager.py, per-row form) as the attention
    function: the median step time of `steps` steps (after one warm-up) of
    the model with each layer count in `layer_counts`, and from those a
    least-squares line t(L) = t0 + L * t_layer (a step is a fixed part --
    embedding, final norm, LM head, argmax -- plus one part per layer),
    which gives the output tokens/s of the 32-layer model the GPU runs."""
    import numpy as np
    import torch
    from transformers import AttentionInterface

    from oracle import eager

    sea = importlib.import_module("serving-engine_amd")
    threads = host_threads()
    torch.set_num_threads(threads)

    def cpu_attention(module, query, key, value, attention_mask, scaling, **kw):
        kc, vc = kw["cache"].blocks(module.layer_idx)
        q = query[0].transpose(0, 1)
        o = eager.eager_step(q, key[0].transpose(0, 1), value[0].transpose(0, 1), kc, vc, kw["write_index"],
                             kw["rows"], scaling, kc.shape[2], per_row=True)
        return o.unsqueeze(0), None

    AttentionInterface.register("paged|eager_cpu", cpu_attention)

    def step_seconds(layers):
        cfg = _llama_8b_config(layers)
        model = _random_llama(cfg, torch.device("cpu"), "paged|eager_cpu")
        kv = torch.randn(layers, 2, n, 16, 8, 128, dtype=torch.float32).div_(math.sqrt(128)).to(torch.bfloat16)
        cache = sea._PagedKVCache.__new__(sea._PagedKVCache)  # CPU pool: only .blocks() is used here
        cache.kv_cache, cache.num_kv_heads, cache.head_dim = kv, 8, 128
        lens = list(ctx)
        tok = torch.zeros(len(lens), dtype=torch.int64)

        def step():
            nonlocal tok
            rows = [(1, ln + 1, ln, tb) for ln, tb in zip(lens, tables)]
            slots = torch.tensor([tb[ln // 16] * 16 + ln % 16 for ln, tb in zip(lens, tables)], dtype=torch.int64)
            pos = torch.tensor(lens, dtype=torch.int64).view(1, -1)
            with torch.no_grad():
                out = model(input_ids=tok.view(1, -1), position_ids=pos, cache=cache, write_index=slots, rows=rows,
                            use_cache=False)
            tok = out.logits[0].argmax(-1)
            for i in range(len(lens)):
                lens[i] += 1

        step()  # warm-up
        times = []
        for _ in range(steps):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
        del model, kv, cache
        return statistics.median(times)

    counts = sorted(set(int(x) for x in layer_counts))
    meas = [step_seconds(c) for c in counts]
    if len(counts) > 1:
        slope, t0 = np.polyfit(np.array(counts, dtype=np.float64), np.array(meas), 1)
    else:
        slope, t0 = meas[0], 0.0
    t32 = t0 + 32 * slope
    batch = len(ctx)
    return {
        "tokens_per_s_at_32_layers": round(batch / t32, 2),
        "unit": "tokens/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"{', '.join(map(str, counts))}-layer models of the same shape on the host CPU (bf16, torch, "
                  f"{threads} threads), batch {batch}, eager paged attention (per-row form), median of {steps} steps "
                  f"after 1 warm-up each; step time fitted as t0 + L x t_layer and evaluated at 32 layers",
        "ms_per_step_measured": {f"{c}_layers": round(m * 1e3, 2) for c, m in zip(counts, meas)},
        "ms_per_layer_fitted": round(slope * 1e3, 2),
        "ms_fixed_part_fitted": round(t0 * 1e3, 2),
        "ms_per_step_at_32_layers": round(t32 * 1e3, 2),
    }


def prefill_measure(sea, wl, dev, reps, layers=16):
    """One attention call over the prefill rows of the mixed workload, cycled
    over `layers` pools (so a layer's K/V is not still in the Infinity Cache),
    timed with HIP events on the launch stream; the whole mixed batch too."""
    import dataclasses

    import torch

    full = wl.make_workload(3)
    rows = dataclasses.replace(full, rows=[r for r in full.rows if r.prefill])
    decode = dataclasses.replace(full, rows=[r for r in full.rows if not r.prefill])
    out = {}
    for key, w in (("prefill_rows", rows), ("decode_rows", decode), ("mixed_batch", full)):
        t = wl.make_tensors(w, dev, num_layers=layers, layout=POOL_LAYOUT[DEFAULT_POOL])
        cache = sea._PagedKVCache(t.kv_cache)
        meta = sea.build_paged_batch_metadata(w.scheduler_output(), device=dev)
        blocks = [cache.blocks(i) for i in range(layers)]
        scale = 1.0 / math.sqrt(w.head_dim)

        def run():
            for i in range(layers):
                sea.paged_flash_attention(t.q, blocks[i][0], blocks[i][1], meta, w.num_q_heads,
                                          w.num_kv_heads, scale)

        run()
        torch.cuda.synchronize()
        out[key] = median_pass_us(run, reps) / layers
        del t, cache, blocks
        torch.cuda.empty_cache()
    flops = rows.prefill_flops()
    tflops = flops / (out["prefill_rows"] * 1e-6) / 1e12
    return {
        "workload": full.name,
        "kernel": "attn_prefill_kernel<BF16,128,2> (8 prefill rows only; 4-wave work-groups, two per CU)",
        "bound": "mfma",
        "flops_per_call": flops,
        "avg_call_us": round(out["prefill_rows"], 3),
        "achieved": round(tflops, 1),
        "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "mixed_batch_call_us": round(out["mixed_batch"], 3),
        "decode_rows": {
            "rows": len(decode.rows),
            "avg_call_us": round(out["decode_rows"], 3),
            "algorithmic_bytes": decode.decode_algorithmic_bytes(),
            "achieved": round(decode.decode_algorithmic_bytes() / (out["decode_rows"] * 1e-6) / 1e9, 2),
            "unit": "GB/s",
            "frac": round(decode.decode_algorithmic_bytes() / (out["decode_rows"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "timing": f"median over {reps} passes of {layers} calls, HIP events",
    }


def copy_measure(sea, wl, dev, reps, layers=32, per_rep=4):
    """kvhot_copy_blocks for the prefix-sharing workload's copy-on-write
    pairs (its 256 partially filled last blocks) over a `layers`-layer pool:
    one launch reads and writes every layer's K and V block of each pair.
    Median over `reps` HIP-event timings of `per_rep` back-to-back launches;
    GB/s of read + written bytes against 8 TB/s."""
    import torch

    w = wl.make_workload(4)
    kv = torch.empty(layers, 2, w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, dtype=w.dtype,
                     device=dev)
    kv.view(torch.int16).random_(generator=torch.Generator(device=dev).manual_seed(4))
    cache = sea._PagedKVCache(kv)
    src = torch.as_tensor(w.copy_src, dtype=torch.int64)
    dst = torch.as_tensor(w.copy_dst, dtype=torch.int64)
    cache.copy_blocks(src, dst)  # the pairs are checked once, on the host
    src_d, dst_d = src.to(dev), dst.to(dev)

    def body():
        for _ in range(per_rep):
            cache.copy_blocks(src_d, dst_d, validate=False)

    body()
    us = median_pass_us(body, reps) / per_rep
    block_bytes = w.block_size * w.num_kv_heads * w.head_dim * kv.element_size()
    moved = 2 * len(src) * layers * 2 * block_bytes
    gbs = moved / (us * 1e-6) / 1e9
    del kv, cache
    torch.cuda.empty_cache()
    return {
        "workload": w.name,
        "kernel": "kvhot_copy_blocks",
        "pairs": len(src),
        "layers": layers,
        "bytes_per_launch": moved,
        "median_launch_us": round(us, 3),
        "roofline_us": round(moved / (HBM_PEAK_GBS * 1e3), 3),
        "achieved": round(gbs, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gbs / HBM_PEAK_GBS, 4),
        "timing": f"median over {reps} HIP-event timings of {per_rep} back-to-back launches",
    }


def host_step_cost(sea, w, dev, pt, n=30):
    """Host time per engine step of build_paged_batch_metadata (host arrays,
    one pinned copy, the slot-mapping launch) and of the attention launch
    list (kvhot_paged_attention_schedule and its upload), which one step
    builds once for all its layers: medians of n steps, in microseconds."""
    import torch

    pak = importlib.import_module("serving-engine_amd.paged_attention_kernel")
    lib = importlib.import_module("serving-engine_amd._lib")
    so = w.scheduler_output()
    dtype = lib.dtype_code(w.dtype)
    pt = pak.DEFAULT_PARTITION_TOKENS if pt is None else int(pt)
    tm, tp = [], []
    for _ in range(n + 1):
        t0 = time.perf_counter()
        m = sea.build_paged_batch_metadata(so, device=dev)
        t1 = time.perf_counter()
        pak._schedule(m, dev, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size, pt, True, dtype)
        t2 = time.perf_counter()
        tm.append(t1 - t0)
        tp.append(t2 - t1)
    torch.cuda.synchronize()
    return {"metadata_us": round(statistics.median(tm[1:]) * 1e6, 1),
            "launch_list_us": round(statistics.median(tp[1:]) * 1e6, 1),
            "per": "engine step (both serve every layer of the step)",
            "rows": len(w.rows)}


def cpu_baseline(w, t, layer, budget_s, attn_bytes):
    """The reference's eager path (oracle/eager.py) on this host: append +
    dense masked attention for one layer of the same batch, same values."""
    import torch

    from oracle import eager

    threads = host_threads()
    torch.set_num_threads(threads)
    q = t.q.cpu()
    nk = t.new_k.transpose(1, 2).squeeze(0).cpu()
    nv = t.new_v.transpose(1, 2).squeeze(0).cpu()
    # the reference's eager path views the pool as contiguous [N, 16, Hkv, D]:
    # a pool in another block layout is copied into that one (same values)
    kc0 = t.kv_cache[layer, 0].cpu().contiguous()
    vc0 = t.kv_cache[layer, 1].cpu().contiguous()
    slots = t.slot_mapping.cpu()
    rows = eager.workload_rows(w)
    est = len(w.rows) * w.num_q_heads * sum(x.k_len for x in w.rows) * 4
    per_row = est > 2e9  # whole-batch scores would not fit comfortably
    scale = 1.0 / math.sqrt(w.head_dim)

    def once():
        kc, vc = kc0.clone(), vc0.clone()
        t0 = time.perf_counter()
        eager.eager_step(q, nk, nv, kc, vc, slots, rows, scale, w.num_kv_heads, per_row=per_row)
        return time.perf_counter() - t0

    first = once()  # warm-up
    reps = int(max(1, min(10, (budget_s - first) / max(first, 1e-3))))
    times = [once() for _ in range(reps)]
    sec = statistics.median(times)
    return {
        "value": round(attn_bytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"one layer of the same batch (append + {'per-row' if per_row else 'whole-batch'} dense "
                  f"masked eager attention, bf16, torch CPU), median of {reps} reps after 1 warm-up; "
                  f"{sec * 1e3:.1f} ms per layer",
        "ms_per_layer": round(sec * 1e3, 2),
    }


if __name__ == "__main__":
    main()
