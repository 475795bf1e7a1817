"""Paged attention on MI355X: the drop-in for the reference's
serving_engine/paged_attention_kernel.py.

Same public names, argument order, return values and metadata keys as the
reference:

* ``paged_flash_attention(q, k_cache, v_cache, metadata, num_q_heads,
  num_kv_heads, scale, is_causal=True) -> (o, l)``
  (serving_engine/paged_attention_kernel.py:125-160), computed by the
  hand-written gfx950 kernels of libkvhot (``kvhot_paged_attention``).
* ``build_paged_batch_metadata(scheduler_output, device="cuda") -> dict``
  (serving_engine/paged_attention_kernel.py:163-200).

Differences a caller can see, all additive:

* the metadata dict carries extra keys -- ``max_q_len``, ``max_k_len`` (host
  ints, so no device->host sync per layer), host copies ``host_q_lens``,
  ``host_k_lens``, ``host_q_starts``, ``host_q_pos_offsets``,
  ``host_block_table`` (from which the first attention call
  of a step builds the work-group launch list that every layer then reuses),
  and on a GPU device ``slot_mapping`` / ``positions`` (int64, built on the
  device by ``kvhot_build_slot_mapping``);
* the metadata arrays are views into one device buffer filled by a single
  host->device copy instead of five;
* a query with no visible key yields o = 0 and l = -inf.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .block import BLOCK_SIZE
from .request import is_prefill

PAGED_K_TILE_SIZE = BLOCK_SIZE  # keys per K/V slice (one physical block)
PAGED_Q_TILE_SIZE = 16          # query rows per MFMA tile

# Split-K partition size for decode rows; 0 lets the library choose.
DEFAULT_PARTITION_TOKENS = 0

# Workspaces are per (device, stream): calls sharing one must be stream-ordered.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def schedule_key(device, hq, hkv, d, bs, pt, causal, dtype):
    """Key of a launch list in metadata["_schedules"]: one per attention
    shape (head counts, head_dim, block size, partition size, causality and
    dtype code) on one device."""
    return (hq, hkv, d, bs, pt, bool(causal), dtype, str(device))


def _schedule(metadata, device, hq, hkv, d, bs, pt, causal, dtype):
    """(device units, n_decode, n_prefill, n_merge, workspace bytes, n_prefix)
    of kvhot_paged_attention_schedule for this step, built once per attention
    shape from the host copies of the metadata and cached in the metadata
    dict; None without host copies."""
    host_q = metadata.get("host_q_lens")
    if host_q is None:
        return None
    key = schedule_key(device, hq, hkv, d, bs, pt, causal, dtype)
    cache = metadata.setdefault("_schedules", {})
    if key in cache:
        return cache[key]
    host_k = metadata["host_k_lens"]
    host_off = metadata["host_q_pos_offsets"]
    host_qs = metadata["host_q_starts"]
    host_bt = metadata["host_block_table"]
    lib = _lib.load()
    # decode, prefill, merge units; workspace bytes; shared-prefix units
    counts = [ctypes.c_int64(0) for _ in range(5)]
    args = (host_q.ctypes.data, host_k.ctypes.data, host_qs.ctypes.data, host_off.ctypes.data,
            host_bt.ctypes.data if host_bt.size else None, host_bt.shape[1] if host_bt.ndim == 2 else 0,
            len(host_q), hq, hkv, d, bs, pt, 1 if causal else 0, dtype)
    outs = tuple(ctypes.byref(c) for c in counts)
    total = lib.kvhot_paged_attention_schedule(*args, None, 0, *outs)
    if total < 0:
        _lib.check(int(total), "kvhot_paged_attention_schedule")
    if total == 0:
        hit = None
    else:
        units = torch.empty((total, 8), dtype=torch.int32, pin_memory=True)
        got = lib.kvhot_paged_attention_schedule(*args, units.data_ptr(), total, *outs)
        if got != total:
            _lib.check(-1 if got >= 0 else int(got), "kvhot_paged_attention_schedule")
        hit = (units.to(device, non_blocking=True),) + tuple(int(c.value) for c in counts)
    cache[key] = hit
    return hit


def attn_flags(is_causal: bool, deterministic: bool = False, verify_block_table: bool = False) -> int:
    """attn_flags of the attention entry points (KVHOT_CAUSAL, KVHOT_DETERMINISTIC,
    KVHOT_VERIFY_BLOCKS)."""
    return ((_lib.KVHOT_CAUSAL if is_causal else 0) | (_lib.KVHOT_DETERMINISTIC if deterministic else 0)
            | (_lib.KVHOT_VERIFY_BLOCKS if verify_block_table else 0))


def _host_max(metadata: dict, key: str, src: str) -> int:
    v = metadata.get(key)
    if v is None:
        t = metadata[src]
        v = int(t.max().item()) if t.numel() else 0
    return int(v)


def _check_meta(name: str, t: torch.Tensor, device: torch.device, n: int | None = None) -> None:
    if t.dtype != torch.int32:
        raise TypeError(f"metadata[{name!r}] must be int32, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"metadata[{name!r}] is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"metadata[{name!r}] must be contiguous")
    if n is not None and t.shape[0] != n:
        raise ValueError(f"metadata[{name!r}] has {t.shape[0]} rows, expected {n}")


def paged_flash_attention(q, k_cache, v_cache, metadata, num_q_heads, num_kv_heads, scale,
                          is_causal=True, partition_tokens=None, deterministic=False,
                          verify_block_table=False):
    """Paged attention forward for a ragged batch (serving_engine/paged_attention_kernel.py:125-160).

    q: [total_query, num_q_heads, head_dim] (any strides with unit head_dim
    stride); k_cache / v_cache: [num_blocks, block_size, num_kv_heads,
    head_dim], one layer of the block pool; metadata: the dict of
    build_paged_batch_metadata().  Returns ``o`` shaped and strided like q
    (``torch.empty_like(q)``) and ``l`` = natural-log LSE, fp32
    [total_query, num_q_heads].  Extensions: ``partition_tokens`` cuts
    decode rows into split-K partitions of at most that many keys;
    ``deterministic=True`` makes repeated calls on the same inputs give the
    same bits (decode waves then do not share out slices at run time, which
    costs some speed), as the reference's serial key loop does.
    ``verify_block_table=True`` makes decode waves check the first block of
    their range, which the launch list takes from
    ``metadata["host_block_table"]``, against ``metadata["block_table"]``
    on the device, for callers that edit only the device copy (about 1-2%
    of a decode call).
    """
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("expected q [T, Hq, D] and k_cache/v_cache [N, block_size, Hkv, D]")
    total_query, hq, head_dim = q.shape
    if hq != num_q_heads:
        raise ValueError(f"q has {hq} heads, num_q_heads={num_q_heads}")
    if num_kv_heads <= 0 or num_q_heads % num_kv_heads:
        raise ValueError(f"num_q_heads={num_q_heads} is not a multiple of num_kv_heads={num_kv_heads}")
    if k_cache.shape != v_cache.shape:
        raise ValueError(f"k_cache {tuple(k_cache.shape)} and v_cache {tuple(v_cache.shape)} differ")
    num_blocks, block_size, hkv, dk = k_cache.shape
    if hkv != num_kv_heads or dk != head_dim:
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match Hkv={num_kv_heads}, D={head_dim}")
    if not (q.dtype == k_cache.dtype == v_cache.dtype):
        raise TypeError(f"dtype mismatch: q {q.dtype}, k_cache {k_cache.dtype}, v_cache {v_cache.dtype}")
    device = q.device
    if device.type != "cuda" or k_cache.device != device or v_cache.device != device:
        raise ValueError("q, k_cache and v_cache must be on the same GPU")
    dtype = _lib.dtype_code(q.dtype)

    q_lens = metadata["q_lens"]
    num_rows = q_lens.shape[0]
    o = torch.empty_like(q)
    l = torch.empty((total_query, num_q_heads), dtype=torch.float32, device=device)
    if num_rows == 0 or total_query == 0:
        return o, l
    for name in ("q_lens", "k_lens", "q_starts", "q_pos_offsets"):
        _check_meta(name, metadata[name], device, num_rows)
    bt = metadata["block_table"]
    _check_meta("block_table", bt, device, num_rows)
    bt_stride = int(metadata.get("block_table_row_stride", bt.shape[1] if bt.dim() == 2 else 0))
    max_q = _host_max(metadata, "max_q_len", "q_lens")
    max_k = _host_max(metadata, "max_k_len", "k_lens")
    pt = DEFAULT_PARTITION_TOKENS if partition_tokens is None else int(partition_tokens)

    lib = _lib.load()
    stream = _lib.stream_handle(device)
    plan = _schedule(metadata, device, num_q_heads, num_kv_heads, head_dim, block_size, pt,
                     is_causal, dtype)
    if plan is not None:
        sched, n_dec, n_pre, n_mrg, need, n_pfx = plan
    else:
        sched, n_dec, n_pre, n_mrg, n_pfx = None, 0, 0, 0, 0
        need = lib.kvhot_paged_attention_workspace_bytes(
            num_rows, total_query, max_q, max_k, num_q_heads, num_kv_heads, head_dim,
            block_size, pt, dtype)
        if need < 0:
            _lib.check(int(need), "kvhot_paged_attention_workspace_bytes")
    ws = _workspace(device, stream, need)
    status = lib.kvhot_paged_attention(
        q.data_ptr(), _lib.i64_array(q.stride()),
        k_cache.data_ptr(), _lib.i64_array(k_cache.stride()),
        v_cache.data_ptr(), _lib.i64_array(v_cache.stride()),
        o.data_ptr(), _lib.i64_array(o.stride()),
        l.data_ptr(), _lib.i64_array(l.stride()),
        bt.data_ptr(), bt_stride,
        q_lens.data_ptr(), metadata["k_lens"].data_ptr(),
        metadata["q_starts"].data_ptr(), metadata["q_pos_offsets"].data_ptr(),
        num_rows, total_query, max_q, max_k, num_q_heads, num_kv_heads, head_dim,
        block_size, num_blocks, float(scale), attn_flags(is_causal, deterministic, verify_block_table), dtype, pt,
        sched.data_ptr() if sched is not None else None, n_dec, n_pre, n_mrg, n_pfx,
        need if sched is not None else 0,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        stream)
    _lib.check(status, "kvhot_paged_attention")
    return o, l


def build_paged_batch_metadata(scheduler_output, device="cuda", num_blocks=None):
    """Per-step metadata shared by all layers (serving_engine/paged_attention_kernel.py:163-200).

    Prefill rows: n_q = chunk, n_k = num_computed + chunk, q_pos_offset =
    num_computed; decode rows: n_q = 1, n_k = total_len, q_pos_offset =
    total_len - 1.  Block tables are padded with 0 to the longest row.
    ``num_blocks`` (extension): the pool's block count; the host block tables
    are then checked before anything is copied: a row whose table covers
    fewer than n_k tokens, or names a block outside [0, num_blocks), raises
    IndexError (where the reference's write, index_copy_ at
    serving_engine/model_runner.py:31-32, raises on an out-of-pool slot; the
    append kernel itself skips such slots).
    """
    reqs = scheduler_output.scheduled_requests
    r = len(reqs)
    per_row = np.zeros((4, r), dtype=np.int64)  # q_lens, k_lens, q_starts, q_pos_offsets
    tables = []
    q_start = 0
    for i, req in enumerate(reqs):
        if is_prefill(req):
            n_q = scheduler_output.prefill_chunk_sizes[req.request_id]
            n_k = req.num_computed_tokens + n_q
            off = req.num_computed_tokens
        else:
            n_q = 1
            n_k = req.total_len
            off = req.total_len - 1
        per_row[:, i] = (n_q, n_k, q_start, off)
        tables.append(req.block_table)
        q_start += n_q
    max_blocks = max((len(t) for t in tables), default=0)
    if per_row.size and (per_row.max() > np.iinfo(np.int32).max or per_row.min() < np.iinfo(np.int32).min):
        raise OverflowError("metadata does not fit int32")

    # One host buffer -> one host-to-device copy; the dict values are views.
    host = np.zeros(4 * r + r * max_blocks, dtype=np.int32)
    host[: 4 * r] = per_row.reshape(-1)
    bt_host = host[4 * r:].reshape(r, max_blocks)
    for i, t in enumerate(tables):
        if len(t):
            bt_host[i, : len(t)] = t
    if num_blocks is not None and r:
        need = (per_row[1] + BLOCK_SIZE - 1) // BLOCK_SIZE
        have = np.array([len(t) for t in tables], dtype=np.int64)
        short = np.nonzero(have < need)[0]
        if short.size:
            i = int(short[0])
            raise IndexError(f"row {i}: block table covers {int(have[i]) * BLOCK_SIZE} tokens, "
                             f"the step reads {int(per_row[1, i])}")
        used = bt_host[np.arange(max_blocks)[None, :] < need[:, None]]
        if used.size and (int(used.min()) < 0 or int(used.max()) >= num_blocks):
            bad = int(used.min()) if int(used.min()) < 0 else int(used.max())
            raise IndexError(f"block id {bad} outside the pool [0, {num_blocks})")
    dev = torch.device(device)
    if dev.type == "cuda":
        staged = torch.empty(host.shape[0], dtype=torch.int32, pin_memory=True)
        staged.numpy()[:] = host
        buf = staged.to(dev, non_blocking=True)
    else:
        buf = torch.from_numpy(host).to(dev)
    meta = {
        "q_lens": buf[0:r],
        "k_lens": buf[r:2 * r],
        "q_starts": buf[2 * r:3 * r],
        "q_pos_offsets": buf[3 * r:4 * r],
        "block_table": buf[4 * r:].view(r, max_blocks),
        "block_table_row_stride": max_blocks,
        "total_query": q_start,
        "max_q_len": int(per_row[0].max()) if r else 0,
        "max_k_len": int(per_row[1].max()) if r else 0,
        "host_q_lens": np.ascontiguousarray(host[0:r]),
        "host_k_lens": np.ascontiguousarray(host[r:2 * r]),
        "host_q_starts": np.ascontiguousarray(host[2 * r:3 * r]),
        "host_q_pos_offsets": np.ascontiguousarray(host[3 * r:4 * r]),
        "host_block_table": bt_host,
    }
    if dev.type == "cuda":
        meta["slot_mapping"], meta["positions"] = build_slot_mapping(meta, block_size=BLOCK_SIZE)
    return meta


def build_slot_mapping(metadata, block_size=BLOCK_SIZE, out=None):
    """(slot_mapping, positions), int64 [total_query], built on the device.

    slot = block_table[row, pos // block_size] * block_size + pos % block_size
    for pos = q_pos_offset + i: the write index and RoPE position ids of
    ModelRunner.forward (serving_engine/model_runner.py:127-129, 142-170).
    ``out`` (extension): a (slots, positions) pair of int64 device tensors of
    total_query elements to write instead of new ones.
    """
    bt = metadata["block_table"]
    device = bt.device
    total = int(metadata["total_query"])
    if out is None:
        slots = torch.empty(total, dtype=torch.int64, device=device)
        positions = torch.empty(total, dtype=torch.int64, device=device)
    else:
        slots, positions = out
        for t in out:
            if t.dtype != torch.int64 or t.device != device or t.numel() != total or not t.is_contiguous():
                raise ValueError(f"out tensors must be contiguous int64 [{total}] on {device}")
    r = metadata["q_lens"].shape[0]
    if total == 0 or r == 0:
        return slots, positions
    max_q = _host_max(metadata, "max_q_len", "q_lens")
    lib = _lib.load()
    status = lib.kvhot_build_slot_mapping(
        bt.data_ptr(), int(metadata["block_table_row_stride"]),
        metadata["q_lens"].data_ptr(), metadata["q_starts"].data_ptr(),
        metadata["q_pos_offsets"].data_ptr(), r, total, max_q, block_size,
        slots.data_ptr(), positions.data_ptr(), _lib.stream_handle(device))
    _lib.check(status, "kvhot_build_slot_mapping")
    return slots, positions
