"""The attention parity check (tests/parity.py) rejects wrong answers that
the element-wise bound alone accepts, and accepts a correct bf16 answer.

Wrong answers are made by the oracle itself, on the CPU, from the same seeded
inputs the GPU parity tests use: an all-zero output, one wrong physical block
per row (K and V), every V block swapped for another block's, and on
long rows (32,768 keys, the long-context workload's shape) one 512-key
partition read from the wrong blocks, V only or K and V; and on the
prefill-ring case (every 32-key tile with its own K/V offsets) one tile
computed with the tile its ring slot held before.  A correct answer is
the oracle's with the two roundings a bf16 kernel makes: P rounded to bf16
before the PV product and O rounded to bf16.
"""
import math

import numpy as np
import pytest
import torch

from conftest import sea_module
from oracle import paged_ref
from parity import REL_L2, check_attention, rel_l2, tile_distinct_case


def bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def step_inputs(w):
    """q, and the pools after the step's append, as float32 numpy arrays."""
    wl = sea_module("workloads")
    T = wl.make_tensors(w, "cpu")
    f = lambda t: t.float().numpy()
    kc, vc = paged_ref.reshape_and_cache(f(T.kv_cache[0, 0]), f(T.kv_cache[0, 1]),
                                         f(T.new_k.transpose(1, 2).squeeze(0)),
                                         f(T.new_v.transpose(1, 2).squeeze(0)), T.slot_mapping.numpy())
    return f(T.q), kc, vc


def oracle(w, q, kc, vc, bt=None):
    q_lens, k_lens, q_starts, offs, bt0 = w.arrays()
    return paged_ref.paged_attention(q, kc, vc, q_lens, k_lens, q_starts, offs, bt0 if bt is None else bt,
                                     w.num_q_heads, w.num_kv_heads, 1.0 / math.sqrt(w.head_dim))


def bf16_kernel_model(w, q, kc, vc, rows):
    """Decode rows as a bf16 kernel computes them: fp64 scores, P = exp(s - m)
    rounded to bf16 for the PV product (the row sum from unrounded P), O
    rounded to bf16."""
    q_lens, k_lens, q_starts, offs, bt = w.arrays()
    g = w.num_q_heads // w.num_kv_heads
    out = {}
    for r in rows:
        t, n = int(q_starts[r]), int(k_lens[r])
        k = np.repeat(paged_ref.gather_keys(kc, bt[r], n).astype(np.float64), g, axis=1)
        v = np.repeat(paged_ref.gather_keys(vc, bt[r], n).astype(np.float64), g, axis=1)
        s = np.einsum("hd,nhd->hn", q[t].astype(np.float64), k) / math.sqrt(w.head_dim)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        o = np.einsum("hn,nhd->hd", bf16(p).astype(np.float64), v) / p.sum(axis=1, keepdims=True)
        out[t] = bf16(o)
    return out


@pytest.fixture(scope="module")
def gqa():
    wl = sea_module("workloads")
    w = wl.make_workload(2)
    q, kc, vc = step_inputs(w)
    ref_o, ref_l = oracle(w, q, kc, vc)
    return w, q, kc, vc, ref_o, ref_l


def rejects(o, l, ref_o, ref_l):
    with pytest.raises(AssertionError):
        check_attention(o, l, ref_o, ref_l, torch.bfloat16)


def test_correct_bf16_answer_passes_with_margin(gqa):
    w, q, kc, vc, ref_o, ref_l = gqa
    check_attention(bf16(ref_o), ref_l, ref_o, ref_l, torch.bfloat16)
    model = bf16_kernel_model(w, q, kc, vc, rows=range(0, 64, 8))
    worst = max(float(rel_l2(o, ref_o[t])[0].max()) for t, o in model.items())
    assert worst < REL_L2[torch.bfloat16] / 2, worst
    o = bf16(ref_o)
    for t, x in model.items():
        o[t] = x
    check_attention(o, ref_l, ref_o, ref_l, torch.bfloat16)


def test_element_bound_alone_accepts_zero_output(gqa):
    """Why the L2 bound exists: on values scaled by 1/sqrt(128) the
    element-wise bound passes an all-zero output almost everywhere."""
    _, _, _, _, ref_o, _ = gqa
    within = np.abs(ref_o) <= 2e-2 + 1e-2 * np.abs(ref_o)
    assert within.mean() > 0.99


def test_rejects_all_zero_output(gqa):
    _, _, _, _, ref_o, ref_l = gqa
    rejects(np.zeros_like(ref_o), ref_l, ref_o, ref_l)


def test_rejects_one_wrong_block_per_row(gqa):
    w, q, kc, vc, ref_o, ref_l = gqa
    bt = w.arrays()[4].copy()
    k_lens = w.arrays()[1]
    for r in range(len(bt)):
        nb = math.ceil(int(k_lens[r]) / 16)
        # a block of the next row stands in for this row's middle block
        bt[r, nb // 2] = bt[(r + 1) % len(bt), 0]
    o, l = oracle(w, q, kc, vc, bt)
    rejects(bf16(o), l, ref_o, ref_l)
    # the element-wise bound alone passes it on most rows (the reason for the L2 bound)
    ok_rows = [np.allclose(o[r], ref_o[r], atol=2e-2, rtol=1e-2) for r in range(len(bt))]
    assert np.mean(ok_rows) > 0.9


def test_rejects_every_v_block_swapped(gqa):
    w, q, kc, vc, ref_o, ref_l = gqa
    used = w.used_blocks()
    swapped = vc.copy()
    swapped[used] = vc[np.roll(used, 1)]
    o, l = oracle(w, q, kc, swapped)
    rejects(bf16(o), l, ref_o, ref_l)


@pytest.fixture(scope="module")
def long_rows():
    """Two decode rows of 32,768 keys, 32/8 heads, D=128, N(0,1) values,
    blocks scattered over a pool: the long-context workload's shape."""
    wl = sea_module("workloads")
    rng = np.random.default_rng(1005)
    n = 2 * 2048 + 512
    ids = rng.permutation(n)
    rows = [wl.Row(1, 32768, 32767, ids[i * 2048:(i + 1) * 2048].astype(np.int64), False) for i in range(2)]
    w = wl.Workload(5, "long rows", torch.bfloat16, 32, 8, 128, n, 1.0, rows, partition_tokens=512, seed=1005)
    q, kc, vc = step_inputs(w)
    ref_o, ref_l = oracle(w, q, kc, vc)
    spare = np.setdiff1d(np.arange(n), w.used_blocks())[:32]
    return w, q, kc, vc, ref_o, ref_l, spare


def test_long_rows_correct_answer_passes(long_rows):
    _, _, _, _, ref_o, ref_l, _ = long_rows
    check_attention(bf16(ref_o), ref_l, ref_o, ref_l, torch.bfloat16)


@pytest.mark.parametrize("which", ["v", "kv"])
def test_long_rows_reject_one_wrong_partition(long_rows, which):
    """One 512-key partition (32 blocks) of every row read from other blocks:
    V only (the LSE is then exact, so only the output check can catch it) or
    K and V."""
    w, q, kc, vc, ref_o, ref_l, spare = long_rows
    part = 40  # keys [40 * 512, 41 * 512)
    kb, vb = kc.copy(), vc.copy()
    for x in w.rows:
        blocks = x.block_table[part * 32:(part + 1) * 32]
        vb[blocks] = vc[spare]
        if which == "kv":
            kb[blocks] = kc[spare]
    o, l = oracle(w, q, kb, vb)
    if which == "v":
        np.testing.assert_allclose(l, ref_l, atol=1e-9, rtol=0)
    rejects(bf16(o), l, ref_o, ref_l)


@pytest.fixture(scope="module")
def tile_case():
    wl = sea_module("workloads")
    w, T = tile_distinct_case(wl, 32, 8, 128, "cpu")
    f = lambda t: t.float().numpy()
    kc, vc = paged_ref.reshape_and_cache(f(T.kv_cache[0, 0]), f(T.kv_cache[0, 1]),
                                         f(T.new_k.transpose(1, 2).squeeze(0)),
                                         f(T.new_v.transpose(1, 2).squeeze(0)), T.slot_mapping.numpy())
    q = f(T.q)
    ref_o, ref_l = oracle(w, q, kc, vc)
    return w, q, kc, vc, ref_o, ref_l


def test_tile_distinct_case_correct_answer_passes(tile_case):
    _, _, _, _, ref_o, ref_l = tile_case
    check_attention(bf16(ref_o), ref_l, ref_o, ref_l, torch.bfloat16)


@pytest.mark.parametrize("row,tile", [(0, 40), (1, 70), (4, 20)])
def test_tile_distinct_case_rejects_a_stale_tile(tile_case, row, tile):
    """The prefill-ring parity case (tile-distinct K/V): one 32-key tile of one
    row computed with the tile four earlier (the ring slot's previous
    contents) instead of its own is rejected.  Row 4 is one of the rows that
    share a 64-block prefix, so tile 20 is a prefix tile."""
    w, q, kc, vc, ref_o, ref_l = tile_case
    bt = w.arrays()[4].copy()
    bt[row, 2 * tile:2 * tile + 2] = bt[row, 2 * tile - 8:2 * tile - 6]
    o, l = oracle(w, q, kc, vc, bt)
    rejects(bf16(o), l, ref_o, ref_l)
