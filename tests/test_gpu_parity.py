"""Parity of the HIP hot path (through the C ABI) with the CPU oracle.

KV append, block copy and slot mapping: bit-exact.  Attention: against the
fp64 oracle on identical seeded inputs, within atol 2e-2 / rtol 1e-2 for
bf16/fp16 outputs and 1e-5 for fp32, natural-log LSE within 2e-3 (16-bit) or
1e-5 (fp32), and every (token, head) output vector within a relative L2 error
of 1e-2 (16-bit) or 1e-5 (fp32) (tests/parity.py; tests/test_parity_bound.py
shows that this check rejects one wrong block per row).  Full-size workloads
1-5 run as generated; every case prints its name before touching the GPU.
"""
import dataclasses
import math

import numpy as np
import pytest
import torch

from conftest import load_golden, sea_module
from oracle import eager, paged_ref
from parity import TOL, assert_rel_l2, check_attention, custom, shared_custom, tile_distinct_case

pytestmark = pytest.mark.gpu


def announce(msg):
    print(f"[gpu-case] {msg}", flush=True)


def f32(t):
    return t.float().cpu().numpy()


def bits(t):
    t = t.contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).cpu().numpy()


@pytest.fixture(scope="module")
def wl():
    return sea_module("workloads")


def oracle_step(w, T, rows=None):
    """fp64 oracle of one step (append then attention) from the pre-step
    tensors.  Only the blocks of the checked rows travel to the host: they are
    gathered into a compact pool and the tables and slots are renumbered."""
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    rows = list(range(len(w.rows))) if rows is None else list(rows)
    keep = np.zeros(len(q_lens), dtype=bool)
    keep[rows] = True
    bs = w.block_size
    need = [bt[r, : math.ceil(k_lens[r] / bs)] for r in rows if k_lens[r] > 0]
    used = np.unique(np.concatenate(need)) if need else np.zeros(1, np.int64)
    idx = torch.as_tensor(used, dtype=torch.int64, device=T.kv_cache.device)
    kc = f32(T.kv_cache[0, 0].index_select(0, idx))
    vc = f32(T.kv_cache[0, 1].index_select(0, idx))
    slots = T.slot_mapping.cpu().numpy()
    blk, off = slots // bs, slots % bs
    pos = np.searchsorted(used, blk)
    hit = (pos < len(used)) & (used[np.minimum(pos, len(used) - 1)] == blk)
    new_slots = np.where(hit, pos * bs + off, -1)
    nk = f32(T.new_k.transpose(1, 2).squeeze(0))
    nv = f32(T.new_v.transpose(1, 2).squeeze(0))
    kc, vc = paged_ref.reshape_and_cache(kc, vc, nk, nv, new_slots)
    bt_new = np.searchsorted(used, bt).clip(0, len(used) - 1).astype(np.int32)
    return paged_ref.paged_attention(f32(T.q), kc, vc, np.where(keep, q_lens, 0), k_lens, q_starts, offs,
                                     bt_new, w.num_q_heads, w.num_kv_heads, 1.0 / math.sqrt(w.head_dim))


def hip_step(sea, wl, w, T, partition_tokens=None, meta=None):
    cache = sea._PagedKVCache(T.kv_cache)
    meta = meta if meta is not None else wl.metadata_tensors(w, T.q.device)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    o, l = sea.paged_flash_attention(T.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads,
                                     1.0 / math.sqrt(w.head_dim), partition_tokens=partition_tokens)
    torch.cuda.synchronize()
    return o, l


def assert_attention(w, o, l, ref_o, ref_lse, rows=None):
    o_np, l_np = f32(o), l.cpu().numpy()
    if rows is not None:
        q_lens, _, q_starts, _, _ = w.arrays()
        idx = np.concatenate([np.arange(q_starts[r], q_starts[r] + q_lens[r]) for r in rows])
        o_np, l_np, ref_o, ref_lse = o_np[idx], l_np[idx], ref_o[idx], ref_lse[idx]
    check_attention(o_np, l_np, ref_o, ref_lse, w.dtype)


# ------------------------------------------------------------------ append --

@pytest.mark.parametrize("config", [1, 2, 3])
def test_append_bit_exact(cuda, sea, wl, config):
    w = wl.make_workload(config)
    announce(f"append workload {config}: {w.total_query} tokens")
    T = wl.make_tensors(w, cuda)
    kb, vb = bits(T.kv_cache[0, 0]), bits(T.kv_cache[0, 1])
    nk = bits(T.new_k.transpose(1, 2).squeeze(0))
    nv = bits(T.new_v.transpose(1, 2).squeeze(0))
    sea._PagedKVCache(T.kv_cache).write(T.new_k, T.new_v, 0, T.slot_mapping)
    torch.cuda.synchronize()
    ek, ev = paged_ref.reshape_and_cache(kb, vb, nk, nv, T.slot_mapping.cpu().numpy())
    assert np.array_equal(bits(T.kv_cache[0, 0]), ek)
    assert np.array_equal(bits(T.kv_cache[0, 1]), ev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_append_int32_slots_padding_and_strides(cuda, sea, dtype):
    announce(f"append int32 slots / padding / strided source {dtype}")
    g = torch.Generator(device=cuda).manual_seed(5)
    kv = torch.randn(3, 2, 12, 16, 4, 64, generator=g, device=cuda).to(dtype)
    src = torch.randn(4, 9, 64, generator=g, device=cuda).to(dtype)  # [Hkv, S, D] -> strided view
    key = src.unsqueeze(0)           # [1, Hkv, S, D] with head stride S*D: a non-trivial view
    val = (src * 2).unsqueeze(0)
    slots = torch.tensor([5, -1, 191, 0, 12 * 16, 77, 100, -7, 130], dtype=torch.int32, device=cuda)
    kb, vb = bits(kv[1, 0]), bits(kv[1, 1])
    sea._PagedKVCache(kv).write(key, val, 1, slots)
    torch.cuda.synchronize()
    ek, ev = paged_ref.reshape_and_cache(kb, vb, bits(key[0].transpose(0, 1)), bits(val[0].transpose(0, 1)),
                                         slots.cpu().numpy())
    assert np.array_equal(bits(kv[1, 0]), ek)
    assert np.array_equal(bits(kv[1, 1]), ev)


@pytest.mark.parametrize("layout", ["token-major", "head-major", "kv-interleaved"])
def test_update_writes_then_gathers(cuda, sea, layout):
    """_PagedKVCache.update, the eager path's write then dense gather
    (reference serving_engine/model_runner.py:34-40), on every pool layout:
    the layer's K/V bit-exactly as the oracle's append leaves them, and the
    gathered rows bit-exactly those slots of the flat [N * 16, Hkv, D] view."""
    announce(f"_PagedKVCache.update, {layout} pool")
    g = torch.Generator(device=cuda).manual_seed(17)
    kv = sea.allocate_kv_cache(2, 12, 4, 64, dtype=torch.bfloat16, device=cuda, layout=layout)
    kv.view(torch.int16).random_(generator=g)
    key = torch.randn(1, 4, 7, 64, generator=g, device=cuda).to(torch.bfloat16)
    val = torch.randn(1, 4, 7, 64, generator=g, device=cuda).to(torch.bfloat16)
    write = torch.tensor([3, 17, 18, -1, 100, 191, 0], dtype=torch.int64, device=cuda)
    read = torch.tensor([17, 3, 5, 191, 18, 120, 0, 17], dtype=torch.int64, device=cuda)
    kb, vb = bits(kv[1, 0]), bits(kv[1, 1])
    k_read, v_read = sea._PagedKVCache(kv).update(key, val, 1, read, write)
    torch.cuda.synchronize()
    ek, ev = paged_ref.reshape_and_cache(kb, vb, bits(key[0].transpose(0, 1)), bits(val[0].transpose(0, 1)),
                                         write.cpu().numpy())
    assert np.array_equal(bits(kv[1, 0]), ek) and np.array_equal(bits(kv[1, 1]), ev)
    idx = read.cpu().numpy()
    assert np.array_equal(bits(k_read), ek.reshape(-1, 4, 64)[idx])
    assert np.array_equal(bits(v_read), ev.reshape(-1, 4, 64)[idx])


# ------------------------------------------------------------- block copy --

@pytest.mark.parametrize("bs", [16, 48])
def test_copy_blocks_bit_exact(cuda, sea, wl, bs):
    w = wl.make_workload(4)
    announce(f"copy_blocks {len(w.copy_src)} pairs x 2 layers, block_size {bs}")
    kv = torch.empty(2, 2, w.num_blocks, bs, 8, 128, dtype=torch.bfloat16, device=cuda)
    kv.view(torch.int16).random_(generator=torch.Generator(device=cuda).manual_seed(9))
    before = bits(kv)
    sea._PagedKVCache(kv).copy_blocks(w.copy_src, w.copy_dst)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kv), paged_ref.copy_blocks(before, w.copy_src, w.copy_dst))


def test_copy_blocks_checks_device_ids(cuda, sea):
    """Ids that live on the device are checked too (one host copy) before
    the copy: overlapping or duplicate pairs would race on the device."""
    announce("copy_blocks with device ids")
    kv = torch.zeros(1, 2, 8, 16, 1, 8, device=cuda)
    cache = sea._PagedKVCache(kv)
    ids = lambda x: torch.tensor(x, device=cuda)
    with pytest.raises(ValueError):
        cache.copy_blocks(ids([1, 2]), ids([2, 3]))
    with pytest.raises(ValueError):
        cache.copy_blocks(ids([1, 2]), ids([4, 4]))
    with pytest.raises(IndexError):
        cache.copy_blocks(ids([1]), ids([8]))
    kv[0, 0, 1] = 1.0
    cache.copy_blocks(ids([1]), ids([5]))
    torch.cuda.synchronize()
    assert torch.equal(kv[0, 0, 5], kv[0, 0, 1]) and float(kv[0, 0, 5].min()) == 1.0


# ---------------------------------------------------------- slot mapping --

def test_metadata_and_slot_mapping_on_device(cuda, sea, wl):
    w = wl.make_workload(3)
    announce("build_paged_batch_metadata workload 3 on device")
    so = w.scheduler_output()
    meta = sea.build_paged_batch_metadata(so, device=cuda)
    torch.cuda.synchronize()
    rows = paged_ref.step_rows(so.scheduled_requests, so.prefill_chunk_sizes)
    q_lens, k_lens, q_starts, offs, bt, mb, total = paged_ref.batch_metadata(rows)
    assert meta["q_lens"].cpu().numpy().tolist() == q_lens.tolist()
    assert meta["k_lens"].cpu().numpy().tolist() == k_lens.tolist()
    assert meta["q_starts"].cpu().numpy().tolist() == q_starts.tolist()
    assert meta["q_pos_offsets"].cpu().numpy().tolist() == offs.tolist()
    assert np.array_equal(meta["block_table"].cpu().numpy(), bt)
    assert meta["block_table_row_stride"] == mb and meta["total_query"] == total
    slots, pos = paged_ref.write_slots_and_positions(rows, 16)
    assert np.array_equal(meta["slot_mapping"].cpu().numpy(), slots)
    assert np.array_equal(meta["positions"].cpu().numpy(), pos)
    assert np.array_equal(slots, w.slot_mapping())


# -------------------------------------------------------------- attention --

@pytest.mark.parametrize("name", ["config1_fp32.npz", "gqa_bf16_mixed.npz"])
def test_golden_fixture(cuda, sea, name):
    g = load_golden(name)
    announce(f"golden {name}")
    kv = torch.stack([g["k_cache"], g["v_cache"]]).unsqueeze(0).to(cuda)
    cache = sea._PagedKVCache(kv)
    cache.write(g["new_k"].transpose(0, 1).unsqueeze(0).to(cuda), g["new_v"].transpose(0, 1).unsqueeze(0).to(cuda),
                0, torch.from_numpy(g["slot_mapping"]).to(cuda))
    meta = {k: torch.from_numpy(g[k]).to(cuda) for k in ("q_lens", "k_lens", "q_starts", "q_pos_offsets",
                                                          "block_table")}
    meta["block_table_row_stride"] = g["block_table"].shape[1]
    kc, vc = cache.blocks(0)
    o, l = sea.paged_flash_attention(g["q"].to(cuda), kc, vc, meta, g["num_q_heads"], g["num_kv_heads"],
                                     1.0 / math.sqrt(g["head_dim"]))
    torch.cuda.synchronize()
    live = np.concatenate([np.arange(s, s + n) for s, n in zip(g["q_starts"], g["q_lens"])])
    check_attention(f32(o)[live], l.cpu().numpy()[live], g["expected_o"][live], g["expected_lse"][live],
                    g["dtype"])


def test_config1_fp32(cuda, sea, wl):
    w = wl.make_workload(1)
    announce("attention workload 1 (fp32)")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    o, l = hip_step(sea, wl, w, T)
    assert_attention(w, o, l, ref_o, ref_l)


@pytest.fixture(scope="module")
def config2(cuda, wl):
    w = wl.make_workload(2)
    T = wl.make_tensors(w, cuda)
    snapshot = T.kv_cache.clone()
    ref = oracle_step(w, T)
    return w, T, snapshot, ref


def test_config2_decode(cuda, sea, wl, config2):
    w, T, snap, (ref_o, ref_l) = config2
    announce("attention workload 2 (bf16 GQA decode, 64 rows)")
    T.kv_cache.copy_(snap)
    o, l = hip_step(sea, wl, w, T)
    assert_attention(w, o, l, ref_o, ref_l)
    # same step again: the workspace needs no clearing between calls.  Waves
    # share out slices at run time, so the summation order (and only the last
    # bits) may differ: within 2 bf16 ulps of the first run.
    T.kv_cache.copy_(snap)
    o2, l2 = hip_step(sea, wl, w, T)
    torch.testing.assert_close(o2.float(), o.float(), atol=1e-3, rtol=2 ** -7)
    torch.testing.assert_close(l2, l, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("pt", [None, 256])
def test_config2_without_schedule(cuda, sea, wl, config2, pt):
    """The padded-grid launch a caller gets without host length copies (no
    schedule): device metadata only."""
    w, T, snap, (ref_o, ref_l) = config2
    announce(f"attention workload 2 without a schedule, partition {pt}")
    T.kv_cache.copy_(snap)
    meta = {k: v for k, v in wl.metadata_tensors(w, T.q.device).items() if not k.startswith("host_")}
    o, l = hip_step(sea, wl, w, T, partition_tokens=pt, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)


def test_config2_matches_eager_restatement(cuda, sea, wl, config2):
    """Against the reference's own eager path restated in torch-CPU bf16."""
    w, T, snap, _ = config2
    announce("attention workload 2 vs torch-CPU eager path")
    T.kv_cache.copy_(snap)
    o, _ = hip_step(sea, wl, w, T)
    o_eager = eager.eager_step(T.q.cpu(), T.new_k.transpose(1, 2).squeeze(0).cpu(),
                               T.new_v.transpose(1, 2).squeeze(0).cpu(), snap[0, 0].cpu(), snap[0, 1].cpu(),
                               T.slot_mapping.cpu(), eager.workload_rows(w), 1.0 / math.sqrt(128), 8)
    np.testing.assert_allclose(f32(o), o_eager.float().numpy(), **TOL[torch.bfloat16])
    assert_rel_l2(f32(o), o_eager.float().numpy(), torch.bfloat16, what="o vs eager")


@pytest.mark.parametrize("pt", [32, 64, 128, 256, 512, 1024])
def test_config2_partition_sizes(cuda, sea, wl, config2, pt):
    w, T, snap, (ref_o, ref_l) = config2
    announce(f"attention workload 2, split-K partition {pt}")
    T.kv_cache.copy_(snap)
    o, l = hip_step(sea, wl, w, T, partition_tokens=pt)
    assert_attention(w, o, l, ref_o, ref_l)


def test_config3_mixed_prefill_decode(cuda, sea, wl):
    w = wl.make_workload(3)
    announce("attention workload 3 (8 x 512-token chunks + 56 decode rows)")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    o, l = hip_step(sea, wl, w, T, meta=sea.build_paged_batch_metadata(w.scheduler_output(), device=cuda))
    assert_attention(w, o, l, ref_o, ref_l)


@pytest.mark.parametrize("config,layout", [(2, "head-major"), (3, "head-major"), (2, "kv-interleaved"),
                                           (3, "kv-interleaved"), (4, "kv-interleaved")])
def test_strided_pool_layouts(cuda, sea, wl, config, layout):
    """The pool stored block-wise as [Hkv, 16, D] (head-major) or [Hkv, 2, 16,
    D] (kv-interleaved, allocate_kv_cache's default): same shape and values,
    other strides; append, attention and block copy give what they give on
    the reference's layout."""
    w = wl.make_workload(config)
    announce(f"attention workload {config} on a {layout} pool")
    T = wl.make_tensors(w, cuda, layout=layout)
    heads = 16 * w.head_dim * (2 if layout == "kv-interleaved" else 1)
    assert T.kv_cache.stride()[3:] == (w.head_dim, heads, 1)
    ref_o, ref_l = oracle_step(w, T)
    meta = sea.build_paged_batch_metadata(w.scheduler_output(), device=cuda) if config == 3 else None
    o, l = hip_step(sea, wl, w, T, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)
    # the append landed in the slots bit-exactly
    slots = T.slot_mapping.cpu()
    kc = T.kv_cache[0, 0].reshape(-1, w.num_kv_heads, w.head_dim)
    assert torch.equal(kc[slots.to(cuda)].cpu(), T.new_k.transpose(1, 2).squeeze(0).cpu())
    # block copy moves whole blocks, K and V
    cache = sea._PagedKVCache(T.kv_cache)
    before = T.kv_cache.clone()
    src = int(slots[0]) // 16
    dst = w.num_blocks - 1 if src != w.num_blocks - 1 else w.num_blocks - 2
    cache.copy_blocks([src], [dst])
    torch.cuda.synchronize()
    assert torch.equal(T.kv_cache[:, :, dst], before[:, :, src])
    rest = torch.arange(w.num_blocks, device=cuda) != dst
    assert torch.equal(T.kv_cache[:, :, rest], before[:, :, rest])


def test_config4_prefix_sharing_and_cow(cuda, sea, wl):
    w = wl.make_workload(4)
    announce("attention workload 4 (256 rows sharing 64 blocks) + copy-on-write")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    o, l = hip_step(sea, wl, w, T)
    assert_attention(w, o, l, ref_o, ref_l)
    # copy-on-write: move every row's last block to a fresh copy and re-point the table
    cache = sea._PagedKVCache(T.kv_cache)
    cache.copy_blocks(w.copy_src, w.copy_dst)
    meta = wl.metadata_tensors(w, cuda)
    bt, host_bt = meta["block_table"], meta["host_block_table"]  # the schedule reads the host copy
    for i, x in enumerate(w.rows):
        bt[i, math.ceil(x.k_len / 16) - 1] = int(w.copy_dst[i])
        host_bt[i, math.ceil(x.k_len / 16) - 1] = int(w.copy_dst[i])
    assert torch.equal(bt.cpu(), torch.from_numpy(host_bt))
    kc, vc = cache.blocks(0)
    o2, l2 = sea.paged_flash_attention(T.q, kc, vc, meta, 32, 8, 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    assert_attention(w, o2, l2, ref_o, ref_l)
    torch.testing.assert_close(o2.float(), o.float(), atol=1e-3, rtol=2 ** -7)
    torch.testing.assert_close(l2, l, atol=1e-5, rtol=1e-5)


@pytest.mark.timeout(480)  # the fp64 oracle over 16 rows of 32k keys takes a minute or two on the host
def test_config5_long_context_40gb_pool(cuda, sea, wl):
    w = wl.make_workload(5)
    announce("attention workload 5 (16 x 32768 tokens, 40 GB pool)")
    T = wl.make_tensors(w, cuda)
    # the oracle reads the pre-step pool (it appends itself), four rows at a time
    pre = []
    for c in range(0, 16, 4):
        announce(f"  oracle of rows {c}..{c + 3}")
        pre.append(oracle_step(w, T, rows=range(c, c + 4)))
    o, l = hip_step(sea, wl, w, T, partition_tokens=512)
    assert int(w.used_blocks().max()) * 16 * 8 * 128 >= 2**31  # offsets need 64 bits
    for c, (ref_o, ref_l) in zip(range(0, 16, 4), pre):
        announce(f"  oracle check of rows {c}..{c + 3}")
        assert_attention(w, o, l, ref_o, ref_l, rows=range(c, c + 4))
    assert torch.isfinite(o.float()).all() and torch.isfinite(l).all()


# -------------------------------------------------------- shape coverage --

MIXED = [(1, 17, 16), (20, 50, 30), (1, 1, 0), (0, 16, 16), (3, 3, 0), (1, 33, 32), (40, 40, 0),
         (1, 700, 699), (9, 300, 291)]

SHAPES = [
    (32, 8, 128, torch.bfloat16), (8, 8, 128, torch.bfloat16), (16, 8, 128, torch.bfloat16),
    (64, 8, 128, torch.bfloat16), (32, 2, 128, torch.bfloat16), (32, 8, 64, torch.bfloat16),
    (16, 4, 256, torch.bfloat16), (32, 8, 128, torch.float16), (12, 4, 96, torch.bfloat16),
    (32, 8, 128, torch.float32), (12, 12, 64, torch.float32), (24, 8, 128, torch.bfloat16),
    # query groups of 8 and 16 heads at head_dim 256 (the decode work-group's
    # LDS above 64 KiB: 132 and 148 KB) and of 16 heads at head_dim 64
    (32, 4, 256, torch.bfloat16), (32, 2, 256, torch.bfloat16), (32, 2, 64, torch.bfloat16),
]


def mfma_shape(hq, hkv, d, dtype):
    """Shapes the MFMA kernels take: bf16/fp16, head_dim 64/128/256, query
    groups of 1 to 16 heads (powers of two); the rest run the VALU kernel."""
    return dtype in (torch.bfloat16, torch.float16) and d in (64, 128, 256) and hq // hkv in (1, 2, 4, 8, 16)


@pytest.mark.parametrize("hq,hkv,d,dtype", SHAPES)
def test_shapes_mixed_batch(cuda, sea, wl, hq, hkv, d, dtype):
    w = custom(wl, MIXED, hq, hkv, d, dtype)
    announce(f"mixed batch Hq={hq} Hkv={hkv} D={d} {dtype}")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, T.q.device)
    o, l = hip_step(sea, wl, w, T, partition_tokens=64, meta=meta)
    live = [i for i, x in enumerate(w.rows) if x.q_len > 0]
    assert_attention(w, o, l, ref_o, ref_l, rows=live)
    # the path that ran: a launch list (MFMA kernels) exactly for the MFMA shapes
    plans = [p for p in meta.get("_schedules", {}).values() if p is not None]
    assert bool(plans) == mfma_shape(hq, hkv, d, dtype), (hq, hkv, d, dtype)


# a prefill chunk, 70 decode rows sharing 40 blocks (640 keys; one with a
# single key past them), two rows of their own, four sharing too few keys
SHARED = ([(24, 200, 176)] + [(1, 641 + 23 * i, 640 + 23 * i) for i in range(70)]
          + [(1, 900, 899), (1, 1500, 1499)] + [(1, 300 + i, 299 + i) for i in range(4)])
SHARED_RUNS = [(1, 70, 40), (73, 4, 15)]


@pytest.mark.parametrize("hq,hkv,d,dtype", [
    (32, 8, 128, torch.bfloat16), (8, 8, 128, torch.bfloat16), (32, 8, 64, torch.bfloat16),
    (16, 4, 256, torch.bfloat16), (64, 4, 128, torch.float16), (16, 8, 128, torch.bfloat16),
    (32, 4, 256, torch.bfloat16), (32, 2, 256, torch.bfloat16), (32, 2, 64, torch.bfloat16),
])
def test_shared_prefix_shapes(cuda, sea, wl, hq, hkv, d, dtype):
    """Decode rows sharing their leading blocks: the prefix keys are attended
    once by prefix units and folded into each row's decode; the whole batch
    (prefill chunk and unshared rows included) matches the oracle."""
    w = shared_custom(wl, SHARED, SHARED_RUNS, hq, hkv, d, dtype)
    announce(f"shared prefix Hq={hq} Hkv={hkv} D={d} {dtype}")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, cuda)
    o, l = hip_step(sea, wl, w, T, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)
    (plan,) = [p for p in meta["_schedules"].values() if p is not None]
    assert plan[5] > 0  # prefix units ran


def test_non_causal(cuda, sea, wl):
    w = custom(wl, [(5, 40, 0), (1, 100, 50), (33, 33, 0)], 32, 8, 128, torch.bfloat16)
    announce("non-causal")
    T = wl.make_tensors(w, cuda)
    cache = sea._PagedKVCache(T.kv_cache)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    o, l = sea.paged_flash_attention(T.q, kc, vc, wl.metadata_tensors(w, cuda), 32, 8,
                                     1.0 / math.sqrt(128), is_causal=False, partition_tokens=32)
    torch.cuda.synchronize()
    kcn, vcn = f32(T.kv_cache[0, 0]), f32(T.kv_cache[0, 1])
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    ref_o, ref_l = paged_ref.paged_attention(f32(T.q), kcn, vcn, q_lens, k_lens, q_starts, offs, bt, 32, 8,
                                             1.0 / math.sqrt(128), is_causal=False)
    check_attention(f32(o), l.cpu().numpy(), ref_o, ref_l, torch.bfloat16)


def test_strided_query_and_empty_key_row(cuda, sea, wl):
    w = custom(wl, [(1, 50, 49), (4, 20, 16), (1, 0, -1)], 32, 8, 128, torch.bfloat16)
    announce("strided q view + row without keys")
    T = wl.make_tensors(w, cuda)
    # q as HF hands it over: [1, Hq, S, D] transposed view -> [S, Hq, D] non-contiguous
    q_hsd = T.q.transpose(0, 1).contiguous()
    q = q_hsd.transpose(0, 1)
    assert not q.is_contiguous()
    cache = sea._PagedKVCache(T.kv_cache)
    kc, vc = cache.blocks(0)
    o, l = sea.paged_flash_attention(q, kc, vc, wl.metadata_tensors(w, cuda), 32, 8, 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    assert o.stride() == q.stride()
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    ref_o, ref_l = paged_ref.paged_attention(f32(T.q), f32(T.kv_cache[0, 0]), f32(T.kv_cache[0, 1]),
                                             q_lens, k_lens, q_starts, offs, bt, 32, 8, 1.0 / math.sqrt(128))
    check_attention(f32(o), l.cpu().numpy(), ref_o, ref_l, torch.bfloat16)
    assert (f32(o)[5] == 0).all() and np.isneginf(l.cpu().numpy()[5]).all()


def test_hf_attention_adapter(cuda, sea, wl):
    w = custom(wl, [(1, 70, 69), (12, 30, 18), (1, 17, 16)], 32, 8, 128, torch.bfloat16)
    announce("HF attention adapter")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = sea.build_paged_batch_metadata(w.scheduler_output(), device=cuda)

    class Module:
        layer_idx = 0

    query = T.q.transpose(0, 1).unsqueeze(0)  # [1, Hq, S, D]
    out, weights = sea.hip_paged_attention_forward(
        Module(), query, T.new_k, T.new_v, None, 1.0 / math.sqrt(128),
        cache=sea._PagedKVCache(T.kv_cache), write_index=meta["slot_mapping"], paged_metadata=meta)
    torch.cuda.synchronize()
    assert weights is None and out.shape == (1, w.total_query, 32, 128)
    check_attention(f32(out[0]), None, ref_o, ref_l, torch.bfloat16)


@pytest.mark.parametrize("pattern,scale_sign", [("rising", 1.0), ("falling", 1.0), ("random", -1.0),
                                                ("random", 0.0)])
def test_prefill_softmax_reference_moves(cuda, sea, wl, pattern, scale_sign):
    """Scores that climb by ~33 log2 units per 32-key tile (every tile moves
    the softmax reference past the lazy threshold), scores that fall (later
    probabilities underflow), and negative / zero scales."""
    w = custom(wl, [(100, 400, 300), (1, 257, 256), (64, 64, 0), (40, 200, 160)], 32, 8, 128,
               torch.bfloat16)
    announce(f"prefill softmax reference: {pattern} scores, scale sign {scale_sign}")
    T = wl.make_tensors(w, cuda)
    if pattern != "random":
        gen = torch.Generator(device=cuda)
        gen.manual_seed(7)
        u = torch.randn(128, generator=gen, device=cuda)
        u = u / u.norm()
        for row in w.rows:
            j = torch.arange(row.k_len, device=cuda)
            ramp = 2.0 * (j if pattern == "rising" else row.k_len - j).float()
            blocks = torch.as_tensor(row.block_table, device=cuda)[j // 16]
            kslice = T.kv_cache[0, 0, blocks, j % 16].float()  # [k_len, Hkv, D]
            T.kv_cache[0, 0, blocks, j % 16] = (kslice + ramp[:, None, None] * u).to(T.kv_cache.dtype)
        T.q.copy_((T.q.float() + 4.0 * u).to(T.q.dtype))
    scale = scale_sign / math.sqrt(128)
    kc, vc = sea._PagedKVCache(T.kv_cache).blocks(0)
    o, l = sea.paged_flash_attention(T.q, kc, vc, wl.metadata_tensors(w, cuda), 32, 8, scale)
    torch.cuda.synchronize()
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    ref_o, ref_l = paged_ref.paged_attention(f32(T.q), f32(T.kv_cache[0, 0]), f32(T.kv_cache[0, 1]),
                                             q_lens, k_lens, q_starts, offs, bt, 32, 8, scale)
    check_attention(f32(o), None, ref_o, ref_l, torch.bfloat16)
    np.testing.assert_allclose(l.cpu().numpy(), ref_l, atol=2e-3, rtol=2e-4)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (32, 8, 64), (16, 4, 256)])
def test_prefill_ring_tiles_distinct(cuda, sea, wl, hq, hkv, d):
    """The prefill kernel's K/V tiles pass through a four-slot LDS ring, filled
    by DMA two or three tiles ahead and ordered by hand-counted waits.  Here
    every 32-key tile's V carries its own direction (a 2.0 offset on head_dim
    (tile mod D)) and its K a smaller one (0.5 on head_dim (tile + 7) mod D),
    so a wave that reads a slot before its tile lands, or after the next one
    overwrote it, gets another tile's offsets: relative L2 errors of several
    percent, against about 2e-3 for a correct kernel.  Prefill rows of many
    tiles (long contexts, causal chunks) and shared-prefix units both run."""
    announce(f"prefill ring: tile-distinct K/V, Hq={hq} Hkv={hkv} D={d}")
    w, T = tile_distinct_case(wl, hq, hkv, d, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, cuda)
    o, l = hip_step(sea, wl, w, T, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)
    (plan,) = [p for p in meta["_schedules"].values() if p is not None]
    assert plan[5] > 0 and plan[2] > plan[5]  # prefix units and prefill rows ran


@pytest.mark.parametrize("nrows,shared", [(4, 32), (16, 16)])
def test_long_rows_sharing_a_short_prefix(cuda, sea, wl, nrows, shared):
    """A few 16k-key rows sharing a short prefix: the prefix is attended once
    by prefix units, and the rows' tails are cut across work-groups, their
    merge units folding the prefix partials in as extra inputs (12 inputs per
    unit with 4 rows, about 4 with 16)."""
    spec = [(1, 16384, 16383)] * nrows
    w = shared_custom(wl, spec, [(0, nrows, shared)], 32, 8, 128, torch.bfloat16, seed=31 + nrows)
    announce(f"{nrows} rows x 16384 keys sharing {shared} blocks")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, cuda)
    o, l = hip_step(sea, wl, w, T, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)
    (plan,) = [p for p in meta["_schedules"].values() if p is not None]
    assert plan[5] > 0 and plan[3] > 0  # prefix units, and merge units for the cut tails



@pytest.mark.parametrize("config,scheduled", [(2, True), (2, False), (3, True), (4, True)])
def test_deterministic_calls_repeat_bitwise(cuda, sea, wl, config, scheduled):
    """deterministic=True (KVHOT_DETERMINISTIC): two calls on the same inputs
    give the same bits of out and lse -- decode with and without a launch
    list, a mixed prefill + decode batch, and shared-prefix rows -- and both
    match the oracle."""
    w = wl.make_workload(config)
    announce(f"deterministic attention, workload {config}, launch list={scheduled}")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, cuda)
    if not scheduled:
        meta = {k: v for k, v in meta.items() if not k.startswith("host_")}
    cache = sea._PagedKVCache(T.kv_cache)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    outs = []
    for _ in range(2):
        o, l = sea.paged_flash_attention(T.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads,
                                         1.0 / math.sqrt(w.head_dim), deterministic=True)
        torch.cuda.synchronize()
        outs.append((bits(o), l.cpu().numpy().view(np.int32)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    assert_attention(w, o, l, ref_o, ref_l)


def test_deterministic_cut_rows_repeat_bitwise(cuda, sea, wl):
    """deterministic=True on a plan that cuts rows across work-groups (a few
    long rows: parts joined by the merge launch): two calls give the same
    bits, and match the oracle."""
    w = custom(wl, [(1, 16384, 16383), (1, 12000, 11999), (1, 300, 299)], 32, 8, 128, torch.bfloat16)
    announce("deterministic attention, 3 decode rows of up to 16384 keys (cut plan)")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, cuda)
    cache = sea._PagedKVCache(T.kv_cache)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    outs = []
    for _ in range(2):
        o, l = sea.paged_flash_attention(T.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads,
                                         1.0 / math.sqrt(w.head_dim), deterministic=True)
        torch.cuda.synchronize()
        outs.append((bits(o), l.cpu().numpy().view(np.int32)))
    (plan,) = [p for p in meta["_schedules"].values() if p is not None]
    assert plan[3] > 0  # merge units: the long rows were cut
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    assert_attention(w, o, l, ref_o, ref_l)


@pytest.mark.parametrize("pt", [None, 128])
def test_device_block_table_edit_not_in_the_host_copy(cuda, sea, wl, pt):
    """The launch list carries each decode range's first physical block from
    the host copy of the block table; a caller that then edits only the
    device table (here: rows 0 and 1 swap their first blocks) and passes
    verify_block_table=True (KVHOT_VERIFY_BLOCKS) still gets the attention
    the device table describes: the kernel checks that block against the
    device table before using it.  With 128-token partitions the decode
    work-groups hold several ranges per wave (the other kernel
    instantiation)."""
    w = wl.make_workload(2)
    announce(f"attention workload 2, first blocks of rows 0 and 1 swapped on the device only, partitions {pt}")
    T = wl.make_tensors(w, cuda)
    meta = wl.metadata_tensors(w, cuda)
    bt = meta["block_table"]
    a, b = int(bt[0, 0]), int(bt[1, 0])
    assert a != b
    bt[0, 0], bt[1, 0] = b, a
    rows = [dataclasses.replace(r, block_table=r.block_table.copy()) for r in w.rows]
    rows[0].block_table[0], rows[1].block_table[0] = b, a
    w2 = dataclasses.replace(w, rows=rows)
    ref_o, ref_l = oracle_step(w2, T)
    cache = sea._PagedKVCache(T.kv_cache)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    o, l = sea.paged_flash_attention(T.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads,
                                     1.0 / math.sqrt(w.head_dim), partition_tokens=pt,
                                     verify_block_table=True)
    torch.cuda.synchronize()
    assert_attention(w2, o, l, ref_o, ref_l)


def test_device_block_table_edit_after_a_shared_prefix(cuda, sea, wl):
    """The same for rows that share a prefix: the 256 rows of workload 4
    share their first 64 blocks, attended once by prefix units, and each
    row's decode range starts at its first private block.  Rows 0 and 1 swap
    that block on the device only; with verify_block_table=True the decode
    ranges that fold the prefix partials in check it too."""
    w = wl.make_workload(4)
    announce("attention workload 4, first private blocks of rows 0 and 1 swapped on the device only")
    T = wl.make_tensors(w, cuda)
    meta = wl.metadata_tensors(w, cuda)
    bt = meta["block_table"]
    j = 64  # the first block after the 1024 shared keys
    assert all(x.k_len > 16 * (j + 1) for x in w.rows[:2])
    a, b = int(bt[0, j]), int(bt[1, j])
    assert a != b and int(bt[0, 0]) == int(bt[1, 0])
    bt[0, j], bt[1, j] = b, a
    rows = [dataclasses.replace(r, block_table=r.block_table.copy()) for r in w.rows]
    rows[0].block_table[j], rows[1].block_table[j] = b, a
    w2 = dataclasses.replace(w, rows=rows)
    ref_o, ref_l = oracle_step(w2, T)
    cache = sea._PagedKVCache(T.kv_cache)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    o, l = sea.paged_flash_attention(T.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads,
                                     1.0 / math.sqrt(w.head_dim), verify_block_table=True)
    torch.cuda.synchronize()
    (plan,) = [p for p in meta["_schedules"].values() if p is not None]
    assert plan[5] > 0  # prefix units: the rows' shared blocks were grouped
    assert_attention(w2, o, l, ref_o, ref_l)


def test_deterministic_fixed_partitions_repeat_bitwise(cuda, sea, wl):
    """deterministic=True with fixed 128-token partitions (work-groups of
    several ranges per wave, each wave walking its own in order): two calls
    give the same bits, and match the oracle."""
    w = wl.make_workload(2)
    announce("deterministic attention, workload 2, 128-token partitions")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    meta = wl.metadata_tensors(w, cuda)
    cache = sea._PagedKVCache(T.kv_cache)
    cache.write(T.new_k, T.new_v, 0, T.slot_mapping)
    kc, vc = cache.blocks(0)
    outs = []
    for _ in range(2):
        o, l = sea.paged_flash_attention(T.q, kc, vc, meta, w.num_q_heads, w.num_kv_heads,
                                         1.0 / math.sqrt(w.head_dim), partition_tokens=128, deterministic=True)
        torch.cuda.synchronize()
        outs.append((bits(o), l.cpu().numpy().view(np.int32)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    assert_attention(w, o, l, ref_o, ref_l)


@pytest.mark.parametrize("bs,layout", [(32, "token-major"), (48, "token-major"), (64, "token-major"),
                                       (32, "head-major"), (48, "head-major"), (48, "kv-interleaved"),
                                       (64, "kv-interleaved")])
def test_block_sizes(cuda, sea, wl, bs, layout):
    """Pools of 32-, 48- and 64-token blocks (the MFMA kernels take any
    multiple of 16; a 16-key slice or half-tile then starts inside a block),
    in each pool layout: prefill chunks, decode rows sharing a prefix,
    a long decode row and a short one in one batch, against the oracle."""
    nb = -(-320 // bs)  # shared blocks: at least 320 keys
    spec = [(96, 500, 404), (1, 700, 699), (1, 900, 899), (1, 1200, 1199), (1, 650, 649), (1, 1000, 999),
            (1, 800, 799), (1, 6000, 5999), (1, 40, 39), (33, 33, 0)]
    w = shared_custom(wl, spec, [(1, 6, nb)], 32, 8, 128, torch.bfloat16, seed=40 + bs, bs=bs)
    announce(f"block_size {bs}, {layout} pool: mixed batch with 6 rows sharing {nb} blocks")
    T = wl.make_tensors(w, cuda, layout=layout)
    assert T.kv_cache.shape[3] == bs  # [layers, K/V, blocks, block_size, kv heads, head_dim]
    ref_o, ref_l = oracle_step(w, T)
    kb, vb = bits(T.kv_cache[0, 0]), bits(T.kv_cache[0, 1])
    meta = wl.metadata_tensors(w, cuda)
    o, l = hip_step(sea, wl, w, T, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)
    # the append landed bit-exactly in the bs-token blocks
    ek, ev = paged_ref.reshape_and_cache(kb, vb, bits(T.new_k.transpose(1, 2).squeeze(0)),
                                         bits(T.new_v.transpose(1, 2).squeeze(0)), T.slot_mapping.cpu().numpy())
    assert np.array_equal(bits(T.kv_cache[0, 0]), ek) and np.array_equal(bits(T.kv_cache[0, 1]), ev)
    (plan,) = [p for p in meta["_schedules"].values() if p is not None]
    assert plan[5] > 0 and plan[2] > plan[5]  # prefix units and prefill rows ran


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_size_8_runs_the_valu_kernel(cuda, sea, wl, dtype):
    """8-token blocks (not a multiple of 16) take the VALU kernel: a prefill
    chunk and decode rows against the oracle, the append bit-exact."""
    spec = [(40, 100, 60), (1, 300, 299), (1, 17, 16), (1, 1000, 999)]
    w = custom(wl, spec, 16, 4, 64, dtype, seed=50, bs=8)
    announce(f"block_size 8, {dtype}: VALU kernel")
    T = wl.make_tensors(w, cuda)
    ref_o, ref_l = oracle_step(w, T)
    kb, vb = bits(T.kv_cache[0, 0]), bits(T.kv_cache[0, 1])
    meta = wl.metadata_tensors(w, cuda)
    o, l = hip_step(sea, wl, w, T, meta=meta)
    assert_attention(w, o, l, ref_o, ref_l)
    assert all(p is None for p in meta["_schedules"].values())  # no MFMA launch list
    ek, ev = paged_ref.reshape_and_cache(kb, vb, bits(T.new_k.transpose(1, 2).squeeze(0)),
                                         bits(T.new_v.transpose(1, 2).squeeze(0)), T.slot_mapping.cpu().numpy())
    assert np.array_equal(bits(T.kv_cache[0, 0]), ek) and np.array_equal(bits(T.kv_cache[0, 1]), ev)
