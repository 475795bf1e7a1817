"""bench.py's host-side helpers, on the CPU: the launch description of an
attention call is built from its launch list's unit counts, and the CPU
baseline runs on the strided pools the headline uses."""
import importlib.util
import os

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class _W:
    dtype = torch.bfloat16
    head_dim = 128


def test_launch_list_desc_names_every_launch(bench):
    # (units, n_dec, n_pre, n_mrg, workspace bytes, n_pfx)
    meta = {"_schedules": {"k": (None, 4096, 136, 8, 1234, 128)}}
    d = bench.launch_list_desc(meta, _W())
    assert "128 shared-prefix units" in d and "4096 ranges" in d and "8 units" in d
    assert "attn_prefill_kernel<BF16,128> x 8 units" in d  # 136 prefill units, 128 of them shared-prefix
    assert bench.launch_list_desc({"_schedules": {"k": None}}, _W()).endswith("(no launch list)")
    assert "decode" in bench.launch_list_desc({"_schedules": {"k": (None, 4096, 0, 0, 0, 0)}}, _W())


@pytest.mark.parametrize("layout", ["kv-interleaved", "head-major"])
def test_cpu_baseline_takes_a_strided_pool(bench, layout):
    """The headline's pool is kv-interleaved (a strided view); the reference's
    eager path views its pool as contiguous, so the baseline copies it into
    that layout first."""
    import dataclasses
    import importlib

    wl = importlib.import_module("serving-engine_amd.workloads")
    w = wl.make_workload(2)
    w = dataclasses.replace(w, rows=w.rows[:4])
    t = wl.make_tensors(w, "cpu", num_layers=1, layout=layout)
    assert not t.kv_cache.is_contiguous()
    r = bench.cpu_baseline(w, t, 0, budget_s=0.5, attn_bytes=1e6)
    assert r["value"] > 0 and r["kind"] == "port"


def test_bench_layouts_match_the_allocator(bench):
    import importlib

    sea = importlib.import_module("serving-engine_amd")
    assert bench.DEFAULT_POOL == "kv-interleaved" and set(bench.POOL_LAYOUT.values()) == set(sea.POOL_LAYOUTS)
    assert set(bench.LAYOUT_NAMES) == set(bench.POOL_LAYOUT) == set(bench.OTHER_KEYS)
