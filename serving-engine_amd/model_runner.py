"""KV-cache owner and attention adapter: the hot-path half of the reference's
serving_engine/model_runner.py, running on libkvhot.

* ``_PagedKVCache(kv_cache)`` with ``write`` / ``update`` / ``blocks``
  (serving_engine/model_runner.py:11-45) plus ``copy_blocks`` for
  copy-on-write (no counterpart in the reference).
* ``hip_paged_attention_forward``: the HF attention-interface function, same
  contract as ``triton_paged_attention_forward``
  (serving_engine/model_runner.py:48-59); ``register_attention()`` registers
  it under ``PAGED_HIP_ATTN_IMPL`` (the reference registers its Triton adapter
  at import, :62; here registration is explicit so importing this module
  does not import transformers).
* ``allocate_kv_cache`` / ``num_blocks_for_memory``: the pool of
  serving_engine/model_runner.py:101-125.
* ``step_inputs``: a step's metadata, after its copy-on-write block copies.
* ``forward_step`` / ``sample_step``: ModelRunner.forward and engine.step's
  greedy sampling (serving_engine/model_runner.py:131-212,
  serving_engine/engine.py:92-116) with the logits computed for each row's
  last token only (``logits_to_keep``), the argmax taken on the device and
  one batched host copy of the step's tokens.

Model loading and tokenisation stay with the caller.
"""
from __future__ import annotations

import torch

from . import _lib
from .block import BLOCK_SIZE
from .paged_attention_kernel import build_paged_batch_metadata, paged_flash_attention
from .request import RequestPhase

PAGED_HIP_ATTN_IMPL = "paged|hip"


class _PagedKVCache:
    """Duck-typed cache object over the whole pool
    kv_cache[num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim]."""

    def __init__(self, kv_cache: torch.Tensor):
        if kv_cache.dim() != 6 or kv_cache.shape[1] != 2:
            raise ValueError("kv_cache must be [num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim]")
        self.kv_cache = kv_cache
        self.num_kv_heads = kv_cache.shape[-2]
        self.head_dim = kv_cache.shape[-1]
        self._pool = None      # the pool's launch constants, for write()
        self._strides = {}     # ctypes stride arrays of key/value layouts seen by write()

    def _pool_args(self):
        """(pool, base pointer, layer and K/V byte strides, block/token/head/dim
        strides as a ctypes array, block size, blocks, dtype, dtype code,
        device index), computed once per pool tensor."""
        kv = self.kv_cache
        pool = self._pool
        if pool is None or pool[0] is not kv:
            st, es = kv.stride(), kv.element_size()
            pool = (kv, kv.data_ptr(), st[0] * es, st[1] * es, _lib.i64_array(st[2:]), kv.shape[3], kv.shape[2],
                    kv.dtype, _lib.dtype_code(kv.dtype), kv.get_device())
            self._pool = pool
        return pool

    def _stride_array(self, strides):
        arr = self._strides.get(strides)
        if arr is None:
            if len(self._strides) > 64:
                self._strides.clear()
            arr = self._strides[strides] = _lib.i64_array(strides)
        return arr

    def write(self, key_states, value_states, layer_idx, write_index):
        """Scatter new K/V into their slots: k_cache.view(-1, Hkv, D)[write_index[i]] =
        key_states[0, :, i, :] (serving_engine/model_runner.py:21-32), as one
        kvhot_reshape_and_cache launch for K and V.  key_states/value_states:
        [1, Hkv, S, D]; write_index: int64 (or int32) [S] on the cache device.
        Slots outside the pool are skipped instead of raising.  (The launch
        reads the [S, Hkv, D] views' strides straight from the [1, Hkv, S, D]
        tensors: an engine calls this once per layer per step.)"""
        kv, base, layer_bytes, kv_bytes, cache_strides, bs, nblocks, dtype, code, dev = self._pool_args()
        shape = key_states.shape
        if len(shape) != 4 or shape[0] != 1 or value_states.shape != shape:
            raise ValueError(f"key {tuple(key_states.shape)} / value {tuple(value_states.shape)} must be [1, Hkv, S, D]")
        _, hkv, s, d = shape
        if hkv != self.num_kv_heads or d != self.head_dim:
            raise ValueError(f"key/value heads/dim {hkv}/{d} do not match the cache {self.num_kv_heads}/{self.head_dim}")
        if key_states.dtype != dtype or value_states.dtype != dtype:
            raise TypeError(f"key/value dtype {key_states.dtype} does not match the cache dtype {dtype}")
        if write_index.dim() != 1 or write_index.shape[0] != s:
            raise ValueError(f"write_index must be [{s}], got {tuple(write_index.shape)}")
        if write_index.dtype is not torch.int64 and write_index.dtype is not torch.int32:
            raise TypeError(f"write_index must be int64 or int32, got {write_index.dtype}")
        if key_states.get_device() != dev or value_states.get_device() != dev or write_index.get_device() != dev:
            raise ValueError("key, value, write_index and the cache must be on one GPU")
        if not 0 <= layer_idx < kv.shape[0]:
            raise IndexError(f"layer {layer_idx} outside the pool's {kv.shape[0]} layers")
        if s == 0:
            return
        if not write_index.is_contiguous():
            write_index = write_index.contiguous()
        ks, vs = key_states.stride(), value_states.stride()
        k_cache = base + layer_idx * layer_bytes
        status = _lib.load().kvhot_reshape_and_cache(
            key_states.data_ptr(), self._stride_array((ks[2], ks[1], ks[3])),
            value_states.data_ptr(), self._stride_array((vs[2], vs[1], vs[3])),
            k_cache, cache_strides, k_cache + kv_bytes, cache_strides,
            write_index.data_ptr(), 1 if write_index.dtype is torch.int64 else 0,
            s, hkv, d, bs, nblocks, code, _lib.stream_handle(kv.device))
        if status:
            _lib.check(status, "kvhot_reshape_and_cache")

    def update(self, key_states, value_states, layer_idx, read_index, write_index):
        """Eager path: write, then gather a dense [len(read_index), Hkv, D]
        read tensor (serving_engine/model_runner.py:34-40).  Only the write is
        on the hot path; the gather serves the dense eager attention."""
        self.write(key_states, value_states, layer_idx, write_index)
        # reshape: a view for the reference's layout, a copy for a head-major pool
        k_cache = self.kv_cache[layer_idx, 0].reshape(-1, self.num_kv_heads, self.head_dim)
        v_cache = self.kv_cache[layer_idx, 1].reshape(-1, self.num_kv_heads, self.head_dim)
        return torch.index_select(k_cache, 0, read_index), torch.index_select(v_cache, 0, read_index)

    def blocks(self, layer_idx):
        """This layer's block-structured K and V, [num_blocks, block_size, Hkv, D]
        each (serving_engine/model_runner.py:42-45)."""
        return self.kv_cache[layer_idx, 0], self.kv_cache[layer_idx, 1]

    def copy_blocks(self, src_block_ids, dst_block_ids, validate=True):
        """Copy-on-write data mover: kv_cache[:, :, dst[i]] = kv_cache[:, :, src[i]]
        for every layer, K and V, in one launch.  Ids must lie in the pool,
        destinations must be unique and disjoint from the sources (pairs that
        overlap would race).  Checked on the host before the copy: host ids
        as they are, device ids after one copy to the host (a synchronisation;
        ``validate=False`` skips it for ids the caller has already checked --
        the kernel then skips ids outside the pool)."""
        src = torch.as_tensor(src_block_ids, dtype=torch.int64)
        dst = torch.as_tensor(dst_block_ids, dtype=torch.int64)
        if src.shape != dst.shape or src.dim() != 1:
            raise ValueError("src_block_ids and dst_block_ids must be 1-D of equal length")
        n = self.kv_cache.shape[2]
        if validate and src.numel():
            hs, hd = src.cpu(), dst.cpu()  # host ids as they are; device ids: one synchronising copy
            if int(hs.min()) < 0 or int(hs.max()) >= n or int(hd.min()) < 0 or int(hd.max()) >= n:
                raise IndexError(f"block id out of range [0, {n})")
            d = set(hd.tolist())
            if len(d) != hd.numel():
                raise ValueError("destination block ids must be unique")
            if d & set(hs.tolist()):
                raise ValueError("a destination block is also a source block")
        if src.numel() == 0:
            return
        dev = self.kv_cache.device
        src = src.to(dev, non_blocking=True).contiguous()
        dst = dst.to(dev, non_blocking=True).contiguous()
        kv = self.kv_cache
        es = kv.element_size()
        block_bytes = kv[0, 0, 0].numel() * es
        if _dense(kv[0, 0, 0]):
            # K and V of a block each fill one range: the launch copies both
            kv_bytes = kv.stride(1) * es
        elif _dense(kv[0, :, 0]) and kv[0, :, 0].storage_offset() == kv.storage_offset():
            # a kv-interleaved pool: K and V of a block fill one range together,
            # starting at K's first element; its two halves are copied as "K"
            # and "V"
            kv_bytes = block_bytes
        else:
            raise ValueError("each block's [block_size, Hkv, D] payload, or its K and V together, "
                             "must fill one dense range")
        lib = _lib.load()
        status = lib.kvhot_copy_blocks(
            kv.data_ptr(), kv.shape[0], kv.stride(0) * es, kv_bytes,
            kv.stride(2) * es, block_bytes, n, src.data_ptr(), dst.data_ptr(),
            src.numel(), _lib.stream_handle(dev))
        _lib.check(status, "kvhot_copy_blocks")


def hip_paged_attention_forward(module, query, key, value, attention_mask, scaling, **kwargs):
    """HF attention-interface function (serving_engine/model_runner.py:48-59):
    append this layer's K/V, then paged attention over the block pool.
    query [1, Hq, S, D], key/value [1, Hkv, S, D]; kwargs cache, write_index,
    paged_metadata.  Returns ([1, S, Hq, D], None)."""
    cache: _PagedKVCache = kwargs["cache"]
    cache.write(key, value, module.layer_idx, kwargs["write_index"])
    k_cache_blocks, v_cache_blocks = cache.blocks(module.layer_idx)
    q = query.transpose(1, 2).squeeze(0)  # [S, Hq, D]
    o, _ = paged_flash_attention(
        q, k_cache_blocks, v_cache_blocks, kwargs["paged_metadata"],
        num_q_heads=q.shape[1], num_kv_heads=cache.num_kv_heads,
        scale=scaling, is_causal=True,
    )
    return o.unsqueeze(0), None


def register_attention(name: str = PAGED_HIP_ATTN_IMPL) -> str:
    """Registers hip_paged_attention_forward in transformers' attention
    registry (AttentionInterface.register) and returns the name."""
    from transformers import AttentionInterface

    AttentionInterface.register(name, hip_paged_attention_forward)
    return name


def _dense(t):
    """Whether t's elements fill one dense range of memory in some order of
    its dimensions (a block's payload, or a block's K and V together)."""
    dims = sorted((st, sz) for st, sz in zip(t.stride(), t.shape) if sz > 1)
    span = 1
    for st, sz in dims:
        if st != span:
            return False
        span *= sz
    return True


POOL_LAYOUTS = ("kv-interleaved", "head-major", "token-major")


def allocate_kv_cache(num_layers, num_blocks, num_kv_heads, head_dim, dtype=torch.bfloat16,
                      device="cuda", block_size=BLOCK_SIZE, head_major=None, layout="kv-interleaved"):
    """Zero-filled pool [L, 2, N, block_size, Hkv, D] (serving_engine/model_runner.py:101-110).

    Every layout keeps that shape and indexing (the tensor is a view with the
    layout's strides, and every kvhot entry point takes strides); they differ
    in how a block lies in memory:

    * "kv-interleaved" (the default): block n stores, for each kv head, its
      block_size K rows and then its block_size V rows ([L, N, Hkv, 2,
      block_size, D] in memory), so the K and V of one kv head in one block
      -- what a decode wave reads per slice -- are one contiguous range of
      2 * 2 * block_size * D bytes;
    * "head-major": the K and V pools apart, each block [Hkv, block_size, D];
    * "token-major": the reference's blocks, [block_size, Hkv, D].

    In the reference's order a head's rows sit at a fixed offset inside each
    token's [Hkv, D] row, which on MI355X maps some heads to slower HBM
    channels than others.  Measured on the 64-row GQA decode call: 53.1 us
    token-major, 49.0 head-major, 48.5 kv-interleaved (the 16-row 32k-token
    call: 375 us head-major, 343-356 kv-interleaved).

    head_major (the older keyword): True for "head-major", False for
    "token-major"."""
    if head_major is not None:
        layout = "head-major" if head_major else "token-major"
    shape = dict(dtype=dtype, device=device)
    if layout == "kv-interleaved":
        return torch.zeros(num_layers, num_blocks, num_kv_heads, 2, block_size, head_dim, **shape).permute(
            0, 3, 1, 4, 2, 5)
    if layout == "head-major":
        return torch.zeros(num_layers, 2, num_blocks, num_kv_heads, block_size, head_dim, **shape).transpose(3, 4)
    if layout == "token-major":
        return torch.zeros(num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim, **shape)
    raise ValueError(f"unknown pool layout {layout!r}; one of {POOL_LAYOUTS}")


def num_blocks_for_memory(free_bytes, num_layers, num_kv_heads, head_dim, dtype=torch.bfloat16,
                          gpu_memory_utilization=0.9, block_size=BLOCK_SIZE):
    """Pool size from free memory (serving_engine/model_runner.py:112-125)."""
    es = torch.empty((), dtype=dtype).element_size()
    per_block = 2 * num_layers * block_size * num_kv_heads * head_dim * es
    return int(free_bytes * gpu_memory_utilization) // per_block


def step_inputs(scheduler_output, device="cuda", cache=None):
    """Per-step device inputs of ModelRunner.forward's paged path
    (serving_engine/model_runner.py:142-184): the metadata dict, whose
    ``slot_mapping`` is the write_index and ``positions`` the position ids.
    With ``cache``, the step's copy-on-write pairs
    (scheduler_output.blocks_to_copy, from scheduler.Scheduler) are copied
    first, on the same stream, so the step's appends land in the copies, and
    the step's block tables are checked against the pool (IndexError for a
    block outside it, as the reference's index_copy_ raises on an out-of-pool
    write slot)."""
    copies = getattr(scheduler_output, "blocks_to_copy", None)
    if copies:
        if cache is None:
            raise ValueError("the step has copy-on-write block copies: pass the cache")
        src, dst = zip(*copies)
        cache.copy_blocks(list(src), list(dst))
    meta = build_paged_batch_metadata(scheduler_output, device=device,
                                      num_blocks=cache.kv_cache.shape[2] if cache is not None else None)
    return meta, meta.get("slot_mapping"), meta.get("positions")


def step_token_ids(scheduler_output):
    """The step's input tokens, rows in scheduled order
    (serving_engine/model_runner.py:150-163): a prefill row's chunk of its
    tokens from num_computed_tokens on, a decode row's last output token."""
    toks = []
    for req in scheduler_output.scheduled_requests:
        if req.phase == RequestPhase.NEEDS_PREFILL:
            c0 = req.num_computed_tokens
            toks += req.all_token_ids()[c0:c0 + scheduler_output.prefill_chunk_sizes[req.request_id]]
        else:
            toks.append(req.output_token_ids[-1])
    return toks


def forward_step(model, scheduler_output, cache, device="cuda"):
    """ModelRunner.forward (serving_engine/model_runner.py:131-212) on the
    paged|hip path: the step's copy-on-write copies, metadata, one forward
    over the flattened batch, and the last token's logits of each scheduled
    row, [rows, vocab].  The reference computes logits for every token and
    then keeps one per row (:209-212); here ``logits_to_keep`` names those
    rows' last positions, so the LM head runs on one row per request.  Every
    scheduled row must have at least one query token (the scheduler only
    schedules such rows)."""
    meta, slots, pos = step_inputs(scheduler_output, device, cache)
    ids = torch.tensor([step_token_ids(scheduler_output)], dtype=torch.int64).to(device, non_blocking=True)
    keep = (meta["q_starts"] + meta["q_lens"] - 1).long()
    with torch.no_grad():
        out = model(input_ids=ids, position_ids=pos.view(1, -1), cache=cache, write_index=slots,
                    paged_metadata=meta, use_cache=False, logits_to_keep=keep)
    return out.logits[0]


def sample_step(model, scheduler, cache, device="cuda"):
    """One greedy engine iteration (serving_engine/engine.py:92-116):
    schedule, forward_step, argmax on the device, then a single host copy of
    the step's tokens (the reference reads them back one ``.item()`` per
    request), appended to the requests that produced a real next token.
    Returns (scheduler output, the step's last-token logits)."""
    out = scheduler.schedule()
    if not out.scheduled_requests:
        return out, None
    logits = forward_step(model, out, cache, device)
    tokens = logits.argmax(-1).cpu().tolist()
    for req, tok in zip(out.scheduled_requests, tokens):
        if req.phase == RequestPhase.NEEDS_DECODE or req.request_id in out.prefill_final_chunk:
            req.output_token_ids.append(int(tok))
    scheduler.update_after_step(out)
    return out, logits
