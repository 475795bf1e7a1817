"""Attention parity checks shared by the GPU parity tests and the CPU test
that shows they reject wrong answers (tests/test_parity_bound.py).

Two bounds, both must hold:

* the element-wise bound the parity bar states: atol 2e-2 / rtol 1e-2 for
  bf16/fp16 outputs, 1e-5 for fp32; natural-log LSE within atol 2e-3 (16-bit)
  or 1e-5 (fp32);
* a relative L2 bound per (query token, query head) output vector:
  ||o - ref||_2 <= REL_L2 * ||ref||_2.  On workloads whose values are scaled
  down (N(0,1)/sqrt(128)) or whose rows are long (32k keys), |o| is far below
  the element-wise atol, so that bound alone accepts an all-zero output or a
  row that read one wrong block; this one does not.  A correct bf16 kernel
  sits near 2e-3 here: P rounded to bf16 before the PV product (relative
  2^-9 per term) and O rounded to bf16 on the way out.  An output whose
  reference is zero (no visible key) must be exactly zero.
"""
from __future__ import annotations

import math

import numpy as np
import torch

TOL = {
    torch.bfloat16: dict(atol=2e-2, rtol=1e-2),
    torch.float16: dict(atol=2e-2, rtol=1e-2),
    torch.float32: dict(atol=1e-5, rtol=1e-5),
}
LSE_TOL = {
    torch.bfloat16: dict(atol=2e-3, rtol=1e-4),
    torch.float16: dict(atol=2e-3, rtol=1e-4),
    torch.float32: dict(atol=1e-5, rtol=1e-5),
}
REL_L2 = {torch.bfloat16: 1e-2, torch.float16: 1e-2, torch.float32: 1e-5}


def rel_l2(o, ref):
    """Relative L2 error of each output vector (last axis), and the indices
    (over the leading axes) of vectors whose reference is zero but whose
    output is not."""
    o = np.asarray(o, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.sqrt(((o - ref) ** 2).sum(axis=-1))
    nrm = np.sqrt((ref ** 2).sum(axis=-1))
    zero = nrm == 0
    rel = np.where(zero, 0.0, err / np.where(zero, 1.0, nrm))
    bad_zero = np.argwhere(zero & (err > 0))
    return rel, bad_zero


def assert_rel_l2(o, ref, dtype, what="o"):
    """Every (token, head) vector of o within REL_L2[dtype] of ref."""
    rel, bad_zero = rel_l2(o, ref)
    assert bad_zero.size == 0, f"{what}: nonzero output where the reference is 0 at {bad_zero[:5].tolist()}"
    if rel.size == 0:
        return
    worst = np.unravel_index(int(np.argmax(rel)), rel.shape)
    assert rel[worst] <= REL_L2[dtype], (
        f"{what}: relative L2 error {rel[worst]:.3e} at (token, head) {tuple(int(i) for i in worst)} "
        f"exceeds {REL_L2[dtype]:.0e} (median {float(np.median(rel)):.2e})")


def check_attention(o, lse, ref_o, ref_lse, dtype):
    """o, ref_o: [T, Hq, D]; lse, ref_lse: [T, Hq] (lse may be None); numpy
    arrays.  Raises AssertionError unless o and lse meet both bounds."""
    o = np.asarray(o, dtype=np.float64)
    ref_o = np.asarray(ref_o, dtype=np.float64)
    assert np.isfinite(o).all(), "non-finite output"
    np.testing.assert_allclose(o, ref_o, **TOL[dtype])
    if lse is not None:
        np.testing.assert_allclose(np.asarray(lse), ref_lse, **LSE_TOL[dtype])
    assert_rel_l2(o, ref_o, dtype)


# ---------------------------------------------------------------- cases --

def custom(wl, spec, hq, hkv, d, dtype, seed=3, bs=16):
    """spec: (q_len, k_len, q_pos_offset) rows over a shuffled pool of
    bs-token blocks."""
    rng = np.random.default_rng(seed)
    need = [max(1, math.ceil(k / bs)) for _, k, _ in spec]
    n = sum(need) + 7
    perm = rng.permutation(n)
    rows, k0 = [], 0
    for (ql, kl, off), nb in zip(spec, need):
        rows.append(wl.Row(ql, kl, off, perm[k0:k0 + nb].astype(np.int64), ql != 1))
        k0 += nb
    return wl.Workload(0, "custom", dtype, hq, hkv, d, n, 1.0, rows, seed=seed, block_size=bs)


def shared_custom(wl, spec, share, hq, hkv, d, dtype, seed=5, bs=16):
    """custom() whose rows share leading blocks: share = [(first row, rows,
    blocks)], each such run of rows reading the same first `blocks` physical
    blocks."""
    w = custom(wl, spec, hq, hkv, d, dtype, seed=seed, bs=bs)
    n = w.num_blocks
    extra = sum(nb for _, _, nb in share)
    perm = np.random.default_rng(seed + 1).permutation(extra) + n
    k = 0
    for r0, nrows, nb in share:
        common = perm[k:k + nb].astype(np.int64)
        k += nb
        for x in w.rows[r0:r0 + nrows]:
            assert x.q_pos_offset >= nb * bs  # the row's own token lands past the shared blocks
            x.block_table = np.concatenate([common, x.block_table[nb:]])
    w.num_blocks = n + extra
    return w


def tile_distinct_case(wl, hq, hkv, d, device, seed=21):
    """Prefill rows of many 32-key tiles (long contexts, causal chunks) and
    12 decode rows sharing 64 blocks (shared-prefix units), bf16, whose every
    32-key tile carries its own offsets: V + 2.0 on head_dim (tile mod D), K +
    0.5 on head_dim ((tile + 7) mod D).  A kernel that computes one tile with
    another tile's K/V (a ring slot read before its DMA landed, or after the
    next DMA overwrote it) is off by several percent in relative L2.
    Returns (workload, tensors)."""
    spec = ([(512, 2500, 1988), (300, 3001, 2701), (64, 4096, 4032), (33, 700, 667)]
            + [(1, 1200 + 29 * i, 1199 + 29 * i) for i in range(12)])
    w = shared_custom(wl, spec, [(4, 12, 64)], hq, hkv, d, torch.bfloat16, seed=seed)
    T = wl.make_tensors(w, device)
    done = set()  # a shared block holds the same keys (same tile indices) in every row: bump it once
    for x in w.rows:
        nb = math.ceil(x.k_len / 16)
        fresh = [b for b in range(nb) if int(x.block_table[b]) not in done]
        done.update(int(x.block_table[b]) for b in fresh)
        if not fresh:
            continue
        j = (torch.as_tensor(fresh, device=device)[:, None] * 16 + torch.arange(16, device=device)).view(-1)
        j = j[j < x.k_len]
        blocks = torch.as_tensor(x.block_table, device=device)[j // 16]
        tile = j // 32
        for kvi, amp, shift in ((1, 2.0, 0), (0, 0.5, 7)):
            cur = T.kv_cache[0, kvi, blocks, j % 16].float()  # [keys, Hkv, D]
            cur[torch.arange(j.numel(), device=device), :, (tile + shift) % d] += amp
            T.kv_cache[0, kvi, blocks, j % 16] = cur.to(T.kv_cache.dtype)
    return w, T
