"""One decode step of a Hugging Face causal LM on paged|hip attention,
captured once as a HIP graph and replayed every step.

The reference engine runs the model's forward eagerly each step
(serving_engine/engine.py:92-116 -> serving_engine/model_runner.py:131-212):
per layer, Python dispatches the projections, the KV append and the
attention.  At decode batch sizes that dispatch, not the GPU, sets the step
time.  Here the step's kernels -- slot mapping, every layer's append and
attention, the rest of the forward and the greedy argmax -- are recorded into
one graph.  A step then costs, on the host, the per-step metadata (one
pinned host->device copy), the launch list of the attention calls (built on
the host from the same arrays, one more copy) and one graph launch.

Rows are decode rows only: row i's query token is token i, and its new token
goes to position lens[i] - 1 of its block table.  The graph reads every
per-step input from fixed device buffers, which ``step`` refills before each
replay; the launch list's unit counts are part of the recording, so a step
whose counts differ from the recorded ones records the graph again.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .block import BLOCK_SIZE
from .paged_attention_kernel import build_slot_mapping, schedule_key


class DecodeStepGraph:
    """Greedy decode steps of ``model`` (an HF causal LM whose attention
    implementation is paged|hip) over ``batch`` rows as graph replays.

    cache: the _PagedKVCache the model's attention appends to and reads;
    max_blocks: block-table columns (the longest table any step passes).
    ``tokens`` holds the rows' input tokens and, after each step, the tokens
    it produced (fed to the next step); ``logits`` the last step's logits.
    """

    def __init__(self, model, cache, batch, max_blocks, num_q_heads, num_kv_heads, head_dim,
                 device, dtype=torch.bfloat16, block_size=BLOCK_SIZE, partition_tokens=0):
        if batch <= 0 or max_blocks <= 0:
            raise ValueError("batch and max_blocks must be positive")
        self.model, self.cache = model, cache
        self.r, self.max_blocks, self.block_size = batch, max_blocks, block_size
        self.device = torch.device(device)
        if self.device.index is None:  # the launch-list key names the device index
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.shape = (num_q_heads, num_kv_heads, head_dim, block_size, partition_tokens, True,
                      _lib.dtype_code(dtype))
        r = batch
        n = 4 * r + r * max_blocks
        # Two pinned host buffers in turn: one is refilled while the copy out
        # of the other may still be queued.
        self._host = [torch.zeros(n, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self._units = [None, None]
        self._copied = [None, None]
        self._turn = 0
        self._dev = torch.zeros(n, dtype=torch.int32, device=self.device)
        self.slots = torch.zeros(r, dtype=torch.int64, device=self.device)
        self.positions = torch.zeros(r, dtype=torch.int64, device=self.device)
        self.tokens = torch.zeros(r, dtype=torch.int64, device=self.device)
        self.logits = None
        d = self._dev
        self.meta = {
            "q_lens": d[0:r],
            "k_lens": d[r:2 * r],
            "q_starts": d[2 * r:3 * r],
            "q_pos_offsets": d[3 * r:4 * r],
            "block_table": d[4 * r:].view(r, max_blocks),
            "block_table_row_stride": max_blocks,
            "total_query": r,
            "max_q_len": 1,
            "max_k_len": max_blocks * block_size,
            "slot_mapping": self.slots,
            "positions": self.positions,
        }
        self.graph = None
        self._recorded = None  # unit counts the graph was recorded with
        self._units_dev = None
        self.recordings = 0

    # -- per-step inputs ---------------------------------------------------

    def _fill(self, host, lens, tables):
        r, mb = self.r, self.max_blocks
        lens = np.asarray(lens, dtype=np.int64)
        if lens.shape != (r,) or (lens < 1).any():
            raise ValueError(f"lens must be {r} positive lengths")
        if len(tables) != r:
            raise ValueError(f"{len(tables)} block tables for {r} rows")
        a = host.numpy()
        a[0:r] = 1
        a[r:2 * r] = lens
        a[2 * r:3 * r] = np.arange(r)
        a[3 * r:4 * r] = lens - 1
        bt = a[4 * r:].reshape(r, mb)
        bt[:] = 0
        for i, t in enumerate(tables):
            if len(t) > mb or len(t) * self.block_size < lens[i]:
                raise ValueError(f"row {i}: block table of {len(t)} blocks for length {lens[i]}")
            bt[i, :len(t)] = t
        return a

    def _plan(self, a):
        """Launch list of the step's attention calls from the host arrays."""
        r, mb = self.r, self.max_blocks
        hq, hkv, d, bs, pt, causal, dt = self.shape
        lib = _lib.load()
        cnt = [ctypes.c_int64(0) for _ in range(5)]  # decode, prefill, merge, workspace, prefix
        outs = tuple(ctypes.byref(c) for c in cnt)
        base = a.ctypes.data  # q_lens, k_lens, q_starts, q_pos_offsets, block table: int32 views of `a`
        args = (base, base + 4 * r, base + 8 * r, base + 12 * r, base + 16 * r, mb, r, hq, hkv, d, bs, pt,
                1 if causal else 0, dt)
        total = lib.kvhot_paged_attention_schedule(*args, None, 0, *outs)
        if total < 0:
            _lib.check(int(total), "kvhot_paged_attention_schedule")
        units = torch.empty((max(int(total), 1), 8), dtype=torch.int32, pin_memory=True)
        if total > 0:
            got = lib.kvhot_paged_attention_schedule(*args, units.data_ptr(), total, *outs)
            if got != total:
                _lib.check(-1 if got >= 0 else int(got), "kvhot_paged_attention_schedule")
        return units, tuple(int(c.value) for c in cnt)

    # -- the recorded step -------------------------------------------------

    def _forward(self):
        build_slot_mapping(self.meta, block_size=self.block_size, out=(self.slots, self.positions))
        with torch.no_grad():
            out = self.model(input_ids=self.tokens.view(1, -1), position_ids=self.positions.view(1, -1),
                             cache=self.cache, write_index=self.slots, paged_metadata=self.meta,
                             use_cache=False)
        self.logits = out.logits[0]
        self.tokens.copy_(self.logits.argmax(-1))

    def _record(self, units, counts):
        n_dec, n_pre, n_mrg, need, n_pfx = counts
        self._units_dev = units.to(self.device, non_blocking=True)
        # The attention calls find their launch list here (no host copies
        # are read once it is present).
        self.meta["host_q_lens"] = self._host[0].numpy()[: self.r]
        self.meta["_schedules"] = {
            schedule_key(self.device, *self.shape): (self._units_dev, n_dec, n_pre, n_mrg, need, n_pfx)}
        stream = torch.cuda.current_stream(self.device)
        saved = self.tokens.clone()
        # One eager pass on a side stream first (lazy library set-up and
        # allocations happen outside the recording), then the recording.
        side = torch.cuda.Stream(self.device)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            self._forward()
        stream.wait_stream(side)
        self.tokens.copy_(saved)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._forward()
        self.graph = graph
        self._recorded = counts
        self.recordings += 1

    def step(self, lens, tables):
        """One decode step: row i is a sequence of lens[i] tokens (the newest
        one, tokens[i], at position lens[i] - 1) with block table tables[i].
        Returns ``tokens`` (device int64 [batch]), now the step's output."""
        i = self._turn
        self._turn ^= 1
        if self._copied[i] is not None:
            self._copied[i].synchronize()  # the copy out of this buffer has run
        a = self._fill(self._host[i], lens, tables)
        units, counts = self._plan(a)
        self._units[i] = units
        self._dev.copy_(self._host[i], non_blocking=True)
        if counts != self._recorded:
            self._record(units, counts)
        else:
            self._units_dev.copy_(units, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._copied[i] = ev
        self.graph.replay()
        return self.tokens
