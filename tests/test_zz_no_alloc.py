"""kvhot_paged_attention_noalloc against kvhot_paged_attention, through the C ABI.

The no-alloc variant keeps its split-K partials in the library's static
device scratch instead of a caller workspace, and launches a mixed batch on
the caller's stream only.  Two calls in a row per path, the second on a
smaller batch, each compared with the allocating entry point on the same
inputs: within atol 2e-2 / rtol 1e-2 (bf16 outputs), 2e-3 on the LSE and a
relative L2 error of 1e-2 per (token, head), the bar of every attention
parity test here (decode waves claim slices at run time, so the last bits
can differ from call to call).  The first test makes the process's first
no-alloc call -- the one that looks up the scratch array's address -- under
graph capture, and checks every replay of that graph.
"""
import math

import numpy as np
import pytest
import torch

from conftest import sea_module
from parity import check_attention

pytestmark = pytest.mark.gpu

# (q_len, k_len, q_pos_offset) rows: long decode rows cut into 256-key
# partitions, a prefill chunk (so a scheduled batch has prefill and decode
# work-groups), short rows.
BIG = [(1, 3000, 2999), (1, 5000, 4999), (7, 900, 893), (1, 700, 699), (1, 4100, 4099), (1, 17, 16)]
SMALL = [(1, 1500, 1499), (3, 300, 297), (1, 600, 599)]


def announce(msg):
    print(f"[gpu-case] {msg}", flush=True)


def custom(wl, spec, hq=32, hkv=8, d=128, dtype=torch.bfloat16, seed=11):
    rng = np.random.default_rng(seed)
    need = [max(1, math.ceil(k / 16)) for _, k, _ in spec]
    n = sum(need) + 5
    perm = rng.permutation(n)
    rows, k0 = [], 0
    for (ql, kl, off), nb in zip(spec, need):
        rows.append(wl.Row(ql, kl, off, perm[k0:k0 + nb].astype(np.int64), ql != 1))
        k0 += nb
    return wl.Workload(0, "custom", dtype, hq, hkv, d, n, 1.0, rows, seed=seed)


def call_args(sea, lib, w, T, meta, pt, scheduled):
    """Arguments of one attention call through the C ABI, up to (not
    including) the workspace and stream; with the output tensors and the
    partial bytes the call needs."""
    _lib = sea_module("_lib")
    pak = sea_module("paged_attention_kernel")
    q = T.q
    device = q.device
    kc, vc = sea._PagedKVCache(T.kv_cache).blocks(0)
    hq, hkv, d = w.num_q_heads, w.num_kv_heads, w.head_dim
    dtype = _lib.dtype_code(q.dtype)
    total, rows = q.shape[0], meta["q_lens"].shape[0]
    max_q = int(meta["host_q_lens"].max())
    max_k = int(meta["host_k_lens"].max())
    o = torch.empty_like(q)
    l = torch.empty((total, hq), dtype=torch.float32, device=device)
    if scheduled:
        plan = pak._schedule(meta, device, hq, hkv, d, 16, pt, True, dtype)
        assert plan is not None
        sched, n_dec, n_pre, n_mrg, need, n_pfx = plan
        assert n_pre > 0 and (n_mrg > 0 or n_pfx > 0)  # prefill beside decode, and partials to fold
    else:
        sched, n_dec, n_pre, n_mrg, n_pfx = None, 0, 0, 0, 0
        need = lib.kvhot_paged_attention_workspace_bytes(rows, total, max_q, max_k, hq, hkv, d, 16, pt, dtype)
        assert need > 0
    bt = meta["block_table"]
    common = [q.data_ptr(), _lib.i64_array(q.stride()), kc.data_ptr(), _lib.i64_array(kc.stride()),
              vc.data_ptr(), _lib.i64_array(vc.stride()), o.data_ptr(), _lib.i64_array(o.stride()),
              l.data_ptr(), _lib.i64_array(l.stride()), bt.data_ptr(), bt.shape[1],
              meta["q_lens"].data_ptr(), meta["k_lens"].data_ptr(), meta["q_starts"].data_ptr(),
              meta["q_pos_offsets"].data_ptr(), rows, total, max_q, max_k, hq, hkv, d, 16, kc.shape[0],
              1.0 / math.sqrt(d), 1, dtype, pt, sched.data_ptr() if sched is not None else None,
              n_dec, n_pre, n_mrg, n_pfx, need if sched is not None else 0]
    return common, o, l, need


def attention(sea, lib, w, T, meta, pt, scheduled, noalloc):
    """One attention call through the C ABI; returns (o, lse, partial bytes)."""
    _lib = sea_module("_lib")
    common, o, l, need = call_args(sea, lib, w, T, meta, pt, scheduled)
    stream = _lib.stream_handle(T.q.device)
    if noalloc:
        status = lib.kvhot_paged_attention_noalloc(*common, stream)
    else:
        ws = torch.empty(int(need), dtype=torch.uint8, device=T.q.device)
        status = lib.kvhot_paged_attention(*common, ws.data_ptr(), ws.numel(), stream)
    assert status == 0, lib.kvhot_last_error()
    torch.cuda.synchronize()
    return o, l, need


def same(o, l, ref_o, ref_l):
    assert torch.isfinite(o.float()).all() and torch.isfinite(l).all()
    check_attention(o.float().cpu().numpy(), l.cpu().numpy(), ref_o.float().cpu().numpy(), ref_l.cpu().numpy(),
                    torch.bfloat16)


def test_noalloc_first_call_under_graph_capture(cuda, sea):
    """The process's first no-alloc call is made while torch captures a graph
    (no earlier test calls the no-alloc entry point).  The graph is replayed
    three times, with eager work and synchronisations between the replays;
    every replay must match the allocating entry point."""
    wl = sea_module("workloads")
    _lib = sea_module("_lib")
    lib = _lib.load()
    announce("noalloc: first call inside torch.cuda.graph capture, 3 replays")
    w = custom(wl, BIG)
    T = wl.make_tensors(w, cuda)
    meta = wl.metadata_tensors(w, cuda)
    ref_o, ref_l, need = attention(sea, lib, w, T, meta, 256, True, noalloc=False)
    common, o, l, need2 = call_args(sea, lib, w, T, meta, 256, True)
    assert need2 == need > 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.kvhot_paged_attention_noalloc(*common, _lib.stream_handle(cuda))
    assert status == 0, lib.kvhot_last_error()
    for rep in range(3):
        o.fill_(float("nan"))
        l.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        announce(f"  replay {rep}")
        same(o, l, ref_o, ref_l)


@pytest.mark.parametrize("scheduled", [False, True])
def test_noalloc_matches_the_allocating_entry(cuda, sea, scheduled):
    wl = sea_module("workloads")
    lib = sea_module("_lib").load()
    for name, spec in (("big", BIG), ("small", SMALL)):
        announce(f"noalloc vs paged_attention, {name} batch, scheduled={scheduled}")
        w = custom(wl, spec)
        T = wl.make_tensors(w, cuda)
        meta = wl.metadata_tensors(w, cuda)
        ref_o, ref_l, need = attention(sea, lib, w, T, meta, 256, scheduled, noalloc=False)
        o, l, need2 = attention(sea, lib, w, T, meta, 256, scheduled, noalloc=True)
        assert need2 == need <= sea_module("_lib").NOALLOC_SCRATCH_BYTES
        same(o, l, ref_o, ref_l)


def shared(wl, nrows, ctx0, share_blocks, seed):
    """A prefill chunk and `nrows` decode rows (contexts ctx0, ctx0 + 37, ...)
    whose block tables start with the same `share_blocks` blocks."""
    spec = [(9, 60, 51)] + [(1, ctx0 + 37 * i, ctx0 + 37 * i - 1) for i in range(nrows)]
    w = custom(wl, spec, seed=seed)
    common = w.rows[1].block_table[:share_blocks].copy()
    for x in w.rows[1:]:
        x.block_table = np.concatenate([common, x.block_table[share_blocks:]])
    return w


def test_noalloc_shared_prefix_matches_the_allocating_entry(cuda, sea):
    """Shared-prefix units (their partials folded into the decode rows) in the
    scratch array: a batch, then a smaller one."""
    wl = sea_module("workloads")
    lib = sea_module("_lib").load()
    pak = sea_module("paged_attention_kernel")
    for name, (nrows, ctx0, nb) in (("20 rows sharing 40 blocks", (20, 700, 40)),
                                    ("5 rows sharing 17 blocks", (5, 300, 17))):
        announce(f"noalloc vs paged_attention, shared prefix: {name}")
        w = shared(wl, nrows, ctx0, nb, seed=nrows)
        T = wl.make_tensors(w, cuda)
        meta = wl.metadata_tensors(w, cuda)
        ref_o, ref_l, need = attention(sea, lib, w, T, meta, 0, True, noalloc=False)
        plan = pak._schedule(meta, cuda, 32, 8, 128, 16, 0, True, sea_module("_lib").dtype_code(torch.bfloat16))
        assert plan[5] > 0  # shared-prefix units ran
        o, l, need2 = attention(sea, lib, w, T, meta, 0, True, noalloc=True)
        assert need2 == need <= sea_module("_lib").NOALLOC_SCRATCH_BYTES
        same(o, l, ref_o, ref_l)
