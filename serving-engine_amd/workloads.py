"""Seeded synthetic batches for the five paged-attention workloads.

Lengths and block placement come from ``numpy.random.default_rng(1000 + id)``;
tensor values from a seeded ``torch.Generator``.  Every workload is one engine
step: each scheduled query token appends its own K/V (slot mapping), then
attention reads the rows through their block tables.

 1 fp32 decode: 4 rows, ctx {17, 64, 100, 130}, 12/12 heads, D=64, pool of 64
   blocks (a seeded permutation), one-token append per row.
 2 bf16 GQA decode: 64 rows, ctx U[128, 2048], 32/8 heads, D=128, values
   N(0,1)/sqrt(128), pool 1.25x the blocks needed, shuffled; 64-token append.
 3 bf16 chunked prefill, mixed: 56 decode rows ctx U[256, 2048] and 8 rows
   prefilling a 512-token chunk on prior contexts U[0, 4096]; 32/8, D=128.
 4 bf16 prefix sharing: 256 decode rows whose first 64 blocks (1024 tokens)
   are the same physical blocks, each with a private suffix U[64, 512];
   copy-on-write copies of the 256 partially filled last blocks.
 5 bf16 long context: 16 rows x 32768 tokens, blocks scattered over a pool of
   about 40 GB (610,352 blocks of 64 KiB), 512-token split-K partitions.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from .block import BLOCK_SIZE
from .request import Request, RequestPhase, SchedulerOutput


@dataclass
class Row:
    q_len: int
    k_len: int
    q_pos_offset: int
    block_table: np.ndarray  # int64 physical block ids
    prefill: bool


@dataclass
class Workload:
    config: int
    name: str
    dtype: torch.dtype
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    num_blocks: int
    value_scale: float
    rows: list
    block_size: int = BLOCK_SIZE
    copy_src: np.ndarray | None = None
    copy_dst: np.ndarray | None = None
    partition_tokens: int = 0
    seed: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def total_query(self) -> int:
        return sum(r.q_len for r in self.rows)

    @property
    def max_q_len(self) -> int:
        return max((r.q_len for r in self.rows), default=0)

    @property
    def max_k_len(self) -> int:
        return max((r.k_len for r in self.rows), default=0)

    def arrays(self):
        """(q_lens, k_lens, q_starts, q_pos_offsets, block_table) as int32
        numpy arrays; the block table is padded with 0."""
        r = len(self.rows)
        q_lens = np.array([x.q_len for x in self.rows], dtype=np.int32)
        k_lens = np.array([x.k_len for x in self.rows], dtype=np.int32)
        q_starts = np.zeros(r, dtype=np.int32)
        if r:
            q_starts[1:] = np.cumsum(q_lens)[:-1]
        offs = np.array([x.q_pos_offset for x in self.rows], dtype=np.int32)
        mb = max((len(x.block_table) for x in self.rows), default=0)
        bt = np.zeros((r, mb), dtype=np.int32)
        for i, x in enumerate(self.rows):
            bt[i, : len(x.block_table)] = x.block_table
        return q_lens, k_lens, q_starts, offs, bt

    def slot_mapping(self) -> np.ndarray:
        """int64 write slot of every query token (its own position)."""
        out = []
        bs = self.block_size
        for x in self.rows:
            pos = x.q_pos_offset + np.arange(x.q_len)
            out.append(x.block_table[pos // bs] * bs + pos % bs)
        return np.concatenate(out).astype(np.int64) if out else np.zeros(0, np.int64)

    def used_blocks(self) -> np.ndarray:
        ids = [x.block_table[: math.ceil(x.k_len / self.block_size)] for x in self.rows]
        if self.copy_src is not None:
            ids.append(self.copy_src)
        return np.unique(np.concatenate(ids)) if ids else np.zeros(0, np.int64)

    def kv_bytes_read(self) -> int:
        """Logical K+V bytes attention reads (every row's own keys)."""
        es = torch.empty((), dtype=self.dtype).element_size()
        return sum(x.k_len for x in self.rows) * 2 * self.num_kv_heads * self.head_dim * es

    def unique_kv_bytes_read(self) -> int:
        """K+V bytes of distinct physical tokens read (shared prefixes once)."""
        es = torch.empty((), dtype=self.dtype).element_size()
        seen = set()
        bs = self.block_size
        tokens = 0
        for x in self.rows:
            for j in range(math.ceil(x.k_len / bs)):
                b = int(x.block_table[j])
                n = min(bs, x.k_len - j * bs)
                if b not in seen:
                    seen.add(b)
                    tokens += n
        return tokens * 2 * self.num_kv_heads * self.head_dim * es

    def decode_algorithmic_bytes(self, unique: bool = False) -> int:
        """Algorithmic HBM bytes of one attention call: K/V read + Q in + O out
        + block-table entries read + LSE out."""
        es = torch.empty((), dtype=self.dtype).element_size()
        kv = self.unique_kv_bytes_read() if unique else self.kv_bytes_read()
        t = self.total_query
        qo = 2 * t * self.num_q_heads * self.head_dim * es
        btb = sum(math.ceil(x.k_len / self.block_size) for x in self.rows) * 4
        return kv + qo + btb + t * self.num_q_heads * 4

    def prefill_flops(self) -> int:
        """FLOPs of the prefill rows (q_len >= 2) counting only visible
        (query, key) pairs: 4 * Hq * D per pair (QK^T and PV)."""
        pairs = 0
        for x in self.rows:
            if x.q_len < 2:
                continue
            for i in range(x.q_len):
                pairs += max(0, min(x.k_len, x.q_pos_offset + i + 1))
        return 4 * self.num_q_heads * self.head_dim * pairs

    def append_bytes(self) -> int:
        """Algorithmic bytes of the KV append: read K/V + write K/V + slots."""
        es = torch.empty((), dtype=self.dtype).element_size()
        s = self.total_query
        return 4 * s * self.num_kv_heads * self.head_dim * es + 8 * s

    def scheduler_output(self) -> SchedulerOutput:
        """A SchedulerOutput whose rows reproduce this workload's metadata."""
        out = SchedulerOutput()
        for i, x in enumerate(self.rows):
            rid = f"r{i}"
            if x.prefill:
                req = Request(rid, [0] * (x.q_pos_offset + x.q_len), phase=RequestPhase.NEEDS_PREFILL,
                              block_table=[int(b) for b in x.block_table],
                              num_computed_tokens=x.q_pos_offset)
                out.prefill_chunk_sizes[rid] = x.q_len
            else:
                req = Request(rid, [0] * (x.k_len - 1), output_token_ids=[0],
                              phase=RequestPhase.NEEDS_DECODE,
                              block_table=[int(b) for b in x.block_table],
                              num_computed_tokens=x.k_len - 1)
            out.scheduled_requests.append(req)
        return out


def _assign(rng, need_per_row, num_blocks):
    perm = rng.permutation(num_blocks)
    tables, k = [], 0
    for nb in need_per_row:
        tables.append(perm[k:k + nb].astype(np.int64))
        k += nb
    return tables


def _decode_rows(ctx, tables):
    return [Row(1, int(c), int(c) - 1, t, False) for c, t in zip(ctx, tables)]


def make_workload(config: int, seed: int | None = None) -> Workload:
    seed = 1000 + config if seed is None else seed
    rng = np.random.default_rng(seed)
    bs = BLOCK_SIZE
    if config == 1:
        ctx = [17, 64, 100, 130]
        need = [math.ceil(c / bs) for c in ctx]
        tables = _assign(rng, need, 64)
        return Workload(1, "fp32 decode, 4 rows ctx {17,64,100,130}, 12/12 heads, D=64",
                        torch.float32, 12, 12, 64, 64, 1.0, _decode_rows(ctx, tables), seed=seed)
    if config == 2:
        ctx = rng.integers(128, 2048, size=64, endpoint=True)
        need = [math.ceil(int(c) / bs) for c in ctx]
        n = math.ceil(1.25 * sum(need))
        tables = _assign(rng, need, n)
        return Workload(2, "bf16 GQA decode, 64 rows ctx U[128,2048], 32/8 heads, D=128",
                        torch.bfloat16, 32, 8, 128, n, 1.0 / math.sqrt(128),
                        _decode_rows(ctx, tables), seed=seed)
    if config == 3:
        prior = rng.integers(0, 4096, size=8, endpoint=True)
        dctx = rng.integers(256, 2048, size=56, endpoint=True)
        chunk = 512
        need_d = [math.ceil(int(c) / bs) for c in dctx]
        need_p = [math.ceil((int(p) + chunk) / bs) for p in prior]
        n = math.ceil(1.25 * (sum(need_d) + sum(need_p)))
        tables = _assign(rng, need_d + need_p, n)
        rows = _decode_rows(dctx, tables[:56])
        rows += [Row(chunk, int(p) + chunk, int(p), t, True) for p, t in zip(prior, tables[56:])]
        return Workload(3, "bf16 mixed: 56 decode rows ctx U[256,2048] + 8 x 512-token prefill "
                           "chunks on ctx U[0,4096], 32/8 heads, D=128",
                        torch.bfloat16, 32, 8, 128, n, 1.0, rows, seed=seed)
    if config == 4:
        suffix = rng.integers(64, 512, size=256, endpoint=True)
        prefix_blocks = 64
        need_s = [math.ceil(int(s) / bs) for s in suffix]
        n = math.ceil(1.25 * (prefix_blocks + sum(need_s) + 256))
        perm = rng.permutation(n)
        shared = perm[:prefix_blocks].astype(np.int64)
        k = prefix_blocks
        rows, last = [], []
        for s, nb in zip(suffix, need_s):
            own = perm[k:k + nb].astype(np.int64)
            k += nb
            rows.append(Row(1, 1024 + int(s), 1024 + int(s) - 1, np.concatenate([shared, own]), False))
            last.append(own[-1])
        dst = perm[k:k + 256].astype(np.int64)
        return Workload(4, "bf16 prefix-shared decode: 256 rows share 64 blocks (1024 tokens) + "
                           "suffix U[64,512]; 256 copy-on-write block copies, 32/8 heads, D=128",
                        torch.bfloat16, 32, 8, 128, n, 1.0, rows,
                        copy_src=np.array(last, dtype=np.int64), copy_dst=dst, seed=seed)
    if config == 5:
        n = 610_352  # 610,352 x 64 KiB (K+V of one block) = 40.0 GB
        ctx = [32768] * 16
        need = [c // bs for c in ctx]
        ids = rng.choice(n, size=sum(need), replace=False).astype(np.int64)
        tables = [ids[i * need[0]:(i + 1) * need[0]] for i in range(16)]
        return Workload(5, "bf16 long-context decode: 16 rows x 32768 tokens, pool 40 GB, "
                           "32/8 heads, D=128, 512-token partitions",
                        torch.bfloat16, 32, 8, 128, n, 1.0, _decode_rows(ctx, tables),
                        partition_tokens=512, seed=seed)
    raise ValueError(f"unknown workload {config}")


@dataclass
class Tensors:
    kv_cache: torch.Tensor      # [L, 2, N, bs, Hkv, D]
    q: torch.Tensor             # [T, Hq, D]
    new_k: torch.Tensor         # [1, Hkv, T, D]  (the K states this step appends)
    new_v: torch.Tensor
    slot_mapping: torch.Tensor  # int64 [T]


def make_tensors(w: Workload, device="cuda", num_layers: int = 1, head_major: bool = False,
                 layout: str | None = None) -> Tensors:
    """Pool with every used block filled with seeded N(0,1)*value_scale values
    (other blocks zero), plus Q and the K/V to append.  layout: how the pool
    stores a block (allocate_kv_cache's layouts; the same shape and values
    in each); without it, "head-major" if head_major else the reference's
    "token-major"."""
    from .model_runner import allocate_kv_cache

    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    hkv, d, bs = w.num_kv_heads, w.head_dim, w.block_size
    if layout is None:
        layout = "head-major" if head_major else "token-major"
    kv = allocate_kv_cache(num_layers, w.num_blocks, hkv, d, dtype=w.dtype, device=device, block_size=bs,
                           layout=layout)
    used = torch.as_tensor(w.used_blocks(), dtype=torch.int64, device=device)
    for layer in range(num_layers):
        for kvi in range(2):
            vals = torch.randn(used.numel(), bs, hkv, d, generator=gen, device=device,
                               dtype=torch.float32).mul_(w.value_scale).to(w.dtype)
            kv[layer, kvi].index_copy_(0, used, vals)
            del vals
    t = w.total_query
    q = (torch.randn(t, w.num_q_heads, d, generator=gen, device=device) * w.value_scale).to(w.dtype)
    # [T, Hkv, D] values exposed as the [1, Hkv, T, D] transposed view HF produces
    nk = (torch.randn(t, hkv, d, generator=gen, device=device) * w.value_scale).to(w.dtype)
    nv = (torch.randn(t, hkv, d, generator=gen, device=device) * w.value_scale).to(w.dtype)
    slots = torch.as_tensor(w.slot_mapping(), dtype=torch.int64, device=device)
    return Tensors(kv, q, nk.unsqueeze(0).transpose(1, 2), nv.unsqueeze(0).transpose(1, 2), slots)


def metadata_tensors(w: Workload, device="cuda") -> dict:
    """Metadata dict with the reference's keys (plus max_q_len/max_k_len) built
    straight from the workload arrays."""
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    dev = torch.device(device)
    return {
        "q_lens": torch.from_numpy(q_lens).to(dev),
        "k_lens": torch.from_numpy(k_lens).to(dev),
        "q_starts": torch.from_numpy(q_starts).to(dev),
        "q_pos_offsets": torch.from_numpy(offs).to(dev),
        "block_table": torch.from_numpy(bt).to(dev),
        "block_table_row_stride": bt.shape[1],
        "total_query": w.total_query,
        "max_q_len": w.max_q_len,
        "max_k_len": w.max_k_len,
        "host_q_lens": q_lens,
        "host_k_lens": k_lens,
        "host_q_starts": q_starts,
        "host_q_pos_offsets": offs,
        "host_block_table": bt,
    }
