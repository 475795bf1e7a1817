"""Benchmark of the KV-cache hot path on one MI355X.

A step is one engine decode step's worth of hot-path work for the GQA decode
workload (64 rows, ctx U[128, 2048], 32/8 heads, D=128, bf16, block 16, pool
1.25x shuffled): for each of 32 layers, the 64-token KV append
(kvhot_reshape_and_cache) and the split-K paged decode attention
(kvhot_paged_attention) over that layer's pool.  Each layer has its own
~348 MB pool (11 GB in all), so a layer's K/V is never still resident in the
256 MB Infinity Cache when it is read again.

value = algorithmic bytes moved per step (K/V read + Q in + O out + block
table + LSE out, plus the append's K/V read+write and slots) / step time, in
GB/s (1e9).  prefill = the chunked-prefill rows of the mixed workload (8 x
512-token chunks on contexts U[0, 4096], 32/8 heads, D=128, bf16): one
attention call over them, FLOPs counted over visible (query, key) pairs only,
against the 2.5 PFLOP/s dense bf16 MFMA peak (and the whole mixed batch of
that workload, decode rows included, timed alongside).  roofline = one attention call alone (the decode launch plus the
merge launch for rows split across work-groups): its algorithmic bytes over
its average duration, timed with HIP events on the launch stream across a run
of back-to-back calls; `traffic` = the HBM bytes rocprofv3's FETCH_SIZE and
WRITE_SIZE counters read for the same call, scaled by what they read for a
copy of known size, as recorded in profiles/attention_decode_gqa64_traffic.md
(null when that file is absent).  cpu_baseline = the reference's eager
PyTorch path (restated in oracle/eager.py) on this host's cores, on one layer
of the same batch.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 2]
       python bench.py --copy-probe   # kvhot_copy_blocks of 256 MiB each way
                                      # (counter calibration)
       python bench.py --prefill-only # the prefill measurement alone
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attention_decode_gqa64_traffic.md")


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", type=int, default=2, choices=[2, 3, 4, 5])
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--partition-tokens", type=int, default=0)
    ap.add_argument("--kernel-reps", type=int, default=10, help="passes over all layers for the kernel timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill MFMA measurement")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill measurement (for counter runs); prints its JSON object")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="budget for the CPU baseline sample")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run kvhot_copy_blocks over 256 MiB each way, 5 times (counter calibration)")
    return ap.parse_args()


def recorded_traffic(workload: int):
    """HBM bytes per attention call recorded from the rocprofv3 counter runs
    (a `traffic_bytes_per_call: N` line of TRAFFIC_FILE), for workload 2."""
    if workload != 2 or not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            if line.strip().startswith("traffic_bytes_per_call:"):
                return int(line.split(":", 1)[1].strip())
    return None


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
    if args.prefill_only:
        import torch

        torch.cuda.set_device(0)
        sea = importlib.import_module("serving-engine_amd")
        wl = importlib.import_module("serving-engine_amd.workloads")
        print(json.dumps({"prefill": prefill_measure(sea, wl, torch.device("cuda:0"),
                                                     reps=max(1, args.kernel_reps // 2))}), flush=True)
        return

    import torch

    sea = importlib.import_module("serving-engine_amd")
    wl = importlib.import_module("serving-engine_amd.workloads")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    w = wl.make_workload(args.workload)
    layers = args.layers if args.workload != 5 else 1  # the 40 GB pool is one layer's
    t = wl.make_tensors(w, dev, num_layers=layers)
    cache = sea._PagedKVCache(t.kv_cache)
    meta = sea.build_paged_batch_metadata(w.scheduler_output(), device=dev)
    slots = meta["slot_mapping"]
    scale = 1.0 / math.sqrt(w.head_dim)
    pt = args.partition_tokens or w.partition_tokens or None
    blocks = [cache.blocks(i) for i in range(layers)]

    def attention(i):
        return sea.paged_flash_attention(t.q, blocks[i][0], blocks[i][1], meta, w.num_q_heads,
                                         w.num_kv_heads, scale, partition_tokens=pt)

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

    # Attention kernel alone: back-to-back launches over the layers.
    reps = max(1, args.kernel_reps)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        for i in range(layers):
            attention(i)
    end.record()
    torch.cuda.synchronize()
    attn_us = start.elapsed_time(end) * 1e3 / (reps * layers)
    attn_gbs = attn_bytes / (attn_us * 1e-6) / 1e9

    # Append alone.
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        for i in range(layers):
            cache.write(t.new_k, t.new_v, i, slots)
    end.record()
    torch.cuda.synchronize()
    append_us = start.elapsed_time(end) * 1e3 / (reps * layers)

    prefill = None
    if not args.no_prefill:
        prefill = prefill_measure(sea, wl, dev, reps=max(1, args.kernel_reps // 2))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, t, layer=0, budget_s=args.cpu_seconds, attn_bytes=attn_bytes + append_bytes)

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
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "one attention call: attn_decode_kernel<BF16,128,16> + attn_merge_kernel<BF16,128> "
                      "(rows split across work-groups)",
            "achieved": round(attn_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": recorded_traffic(args.workload),
            "algorithmic_bytes_per_launch": attn_bytes,
            "avg_launch_us": round(attn_us, 3),
        },
        "append": {"avg_launch_us": round(append_us, 3), "algorithmic_bytes": append_bytes,
                   "gbs": round(append_bytes / (append_us * 1e-6) / 1e9, 2)},
        "cpu_baseline": cpu,
    }
    if prefill is not None:
        line["prefill"] = prefill
    print(json.dumps(line), flush=True)


def prefill_measure(sea, wl, dev, reps, layers=16):
    """One attention call over the prefill rows of the mixed workload, cycled
    over `layers` pools (so a layer's K/V is not still in the Infinity Cache),
    timed with HIP events on the launch stream; the whole mixed batch too."""
    import dataclasses

    import torch

    full = wl.make_workload(3)
    rows = dataclasses.replace(full, rows=[r for r in full.rows if r.prefill])
    out = {}
    for key, w in (("prefill_rows", rows), ("mixed_batch", full)):
        t = wl.make_tensors(w, dev, num_layers=layers)
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
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        out[key] = e0.elapsed_time(e1) * 1e3 / (reps * layers)
        del t, cache, blocks
        torch.cuda.empty_cache()
    flops = rows.prefill_flops()
    tflops = flops / (out["prefill_rows"] * 1e-6) / 1e12
    return {
        "workload": full.name,
        "kernel": "attn_prefill_kernel<BF16,128,2> (8 prefill rows only)",
        "bound": "mfma",
        "flops_per_call": flops,
        "avg_call_us": round(out["prefill_rows"], 3),
        "achieved": round(tflops, 1),
        "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "mixed_batch_call_us": round(out["mixed_batch"], 3),
    }


def cpu_baseline(w, t, layer, budget_s, attn_bytes):
    """The reference's eager path (oracle/eager.py) on this host: append +
    dense masked attention for one layer of the same batch, same values."""
    import torch

    from oracle import eager

    threads = torch.get_num_threads()
    q = t.q.cpu()
    nk = t.new_k.transpose(1, 2).squeeze(0).cpu()
    nv = t.new_v.transpose(1, 2).squeeze(0).cpu()
    kc0 = t.kv_cache[layer, 0].cpu()
    vc0 = t.kv_cache[layer, 1].cpu()
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
        "kind": "port",
        "sample": f"one layer of the same batch (append + {'per-row' if per_row else 'whole-batch'} dense "
                  f"masked eager attention, bf16, torch CPU), median of {reps} reps after 1 warm-up; "
                  f"{sec * 1e3:.1f} ms per layer",
        "ms_per_layer": round(sec * 1e3, 2),
    }


if __name__ == "__main__":
    main()
