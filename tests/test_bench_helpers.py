"""bench.py's host-side helpers, on the CPU: the launch description of an
attention call is built from its launch list's unit counts."""
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
    assert "128 shared-prefix units" in d and "4096 waves" in d and "8 units" in d
    assert "attn_prefill_kernel<BF16,128> x 8 units" in d  # 136 prefill units, 128 of them shared-prefix
    assert bench.launch_list_desc({"_schedules": {"k": None}}, _W()).endswith("(no launch list)")
    assert "decode" in bench.launch_list_desc({"_schedules": {"k": (None, 4096, 0, 0, 0, 0)}}, _W())
