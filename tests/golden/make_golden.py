"""Writes the golden fixtures in this directory: seeded inputs and the fp64
oracle's expected outputs for one engine step (KV append, then paged
attention).

* config1_fp32.npz -- the fp32 decode workload: 4 rows, ctx {17, 64, 100, 130},
  12/12 heads, D=64, a 64-block pool, one-token append per row.
* gqa_bf16_mixed.npz -- a small bf16 GQA batch (8/2 heads, D=128) mixing decode
  rows, prefill chunks with a causal offset, a 0-token chunk and ragged tails.

Only blocks the step touches are stored (with their ids).  Arrays of 16-bit
floats are stored as their raw uint16 bits.  Run from the repository root:
    python tests/golden/make_golden.py
"""
import importlib
import math
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import paged_ref  # noqa: E402

wl = importlib.import_module("serving-engine_amd.workloads")
HERE = os.path.dirname(os.path.abspath(__file__))


def small_bf16_workload():
    rng = np.random.default_rng(2024)
    spec = [  # (q_len, k_len, q_pos_offset)
        (1, 17, 16), (20, 50, 30), (1, 100, 99), (0, 16, 16), (3, 3, 0), (1, 33, 32), (37, 37, 0),
    ]
    need = [math.ceil(k / 16) for _, k, _ in spec]
    n = sum(need) + 5
    perm = rng.permutation(n)
    rows, k0 = [], 0
    for (ql, kl, off), nb in zip(spec, need):
        rows.append(wl.Row(ql, kl, off, perm[k0:k0 + nb].astype(np.int64), ql != 1))
        k0 += nb
    return wl.Workload(0, "small bf16 GQA mixed batch", torch.bfloat16, 8, 2, 128, n, 1.0, rows, seed=77)


def raw(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().numpy()


def write_case(name: str, w) -> None:
    t = wl.make_tensors(w, device="cpu")
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    used = w.used_blocks()
    slots = t.slot_mapping.numpy()
    nk = t.new_k.transpose(1, 2).squeeze(0)  # [T, Hkv, D]
    nv = t.new_v.transpose(1, 2).squeeze(0)
    kc = t.kv_cache[0, 0].float().numpy()
    vc = t.kv_cache[0, 1].float().numpy()
    kc2, vc2 = paged_ref.reshape_and_cache(kc, vc, nk.float().numpy(), nv.float().numpy(), slots)
    o, lse = paged_ref.paged_attention(t.q.float().numpy(), kc2, vc2, q_lens, k_lens, q_starts, offs, bt,
                                       w.num_q_heads, w.num_kv_heads, 1.0 / math.sqrt(w.head_dim))
    np.savez_compressed(
        os.path.join(HERE, name),
        dtype=np.array(str(w.dtype).replace("torch.", "")),
        heads=np.array([w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size, w.num_blocks]),
        q=raw(t.q), new_k=raw(nk), new_v=raw(nv), slot_mapping=slots,
        used_blocks=used, k_blocks=raw(t.kv_cache[0, 0][torch.from_numpy(used)]),
        v_blocks=raw(t.kv_cache[0, 1][torch.from_numpy(used)]),
        q_lens=q_lens, k_lens=k_lens, q_starts=q_starts, q_pos_offsets=offs, block_table=bt,
        expected_o=o.astype(np.float32), expected_lse=lse.astype(np.float32),
    )
    print(f"wrote {name}: T={w.total_query} rows={len(w.rows)} used_blocks={len(used)}")


if __name__ == "__main__":
    write_case("config1_fp32.npz", wl.make_workload(1))
    write_case("gqa_bf16_mixed.npz", small_bf16_workload())
