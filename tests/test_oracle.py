"""Pins the CPU oracle (oracle/paged_ref.py, oracle/eager.py) to checks that do
not restate its formulas: torch's scaled_dot_product_attention, logsumexp and
index_copy_, pure-Python brute force on tiny inputs, hand-computed known
answers, closed-form special cases and invariants -- and shows that planted
mistakes in the oracle are caught by those checks."""
import inspect
import math

import numpy as np
import pytest
import torch

from oracle import eager, paged_ref

BS = 16


def _random_problem(seed, hq, hkv, d, rows_spec, pool=None):
    """rows_spec: list of (q_len, k_len, q_pos_offset)."""
    rng = np.random.default_rng(seed)
    need = [math.ceil(k / BS) for _, k, _ in rows_spec]
    n = pool or sum(need) + 3
    perm = rng.permutation(n)
    tables, k0 = [], 0
    for nb in need:
        tables.append(perm[k0:k0 + nb])
        k0 += nb
    t = sum(q for q, _, _ in rows_spec)
    q = rng.standard_normal((t, hq, d))
    kc = rng.standard_normal((n, BS, hkv, d))
    vc = rng.standard_normal((n, BS, hkv, d))
    q_lens = np.array([r[0] for r in rows_spec], np.int32)
    k_lens = np.array([r[1] for r in rows_spec], np.int32)
    offs = np.array([r[2] for r in rows_spec], np.int32)
    q_starts = np.concatenate([[0], np.cumsum(q_lens)[:-1]]).astype(np.int32)
    mb = max(need)
    bt = np.zeros((len(rows_spec), mb), np.int32)
    for i, tb in enumerate(tables):
        bt[i, : len(tb)] = tb
    return dict(q=q, k_cache=kc, v_cache=vc, q_lens=q_lens, k_lens=k_lens, q_starts=q_starts,
                q_pos_offsets=offs, block_table=bt, num_q_heads=hq, num_kv_heads=hkv,
                scale=1.0 / math.sqrt(d))


def _sdpa_check(p, fn=paged_ref.paged_attention, causal=True):
    """Independent computation with torch SDPA (fp64) + torch.logsumexp."""
    o, lse = fn(**p, is_causal=causal)
    hq, hkv = p["num_q_heads"], p["num_kv_heads"]
    g = hq // hkv
    for r in range(len(p["q_lens"])):
        n_q, n_k, qs, off = (int(p["q_lens"][r]), int(p["k_lens"][r]), int(p["q_starts"][r]),
                             int(p["q_pos_offsets"][r]))
        if n_q == 0:
            continue
        # walk the block table token by token
        ks = np.stack([p["k_cache"][p["block_table"][r][j // BS], j % BS] for j in range(n_k)])
        vs = np.stack([p["v_cache"][p["block_table"][r][j // BS], j % BS] for j in range(n_k)])
        kh = torch.tensor(np.stack([ks[:, h // g] for h in range(hq)]))[None]  # [1, Hq, n_k, D]
        vh = torch.tensor(np.stack([vs[:, h // g] for h in range(hq)]))[None]
        qh = torch.tensor(p["q"][qs:qs + n_q]).transpose(0, 1)[None]          # [1, Hq, n_q, D]
        mask = torch.ones(n_q, n_k, dtype=torch.bool)
        if causal:
            mask = torch.tensor([[j <= off + i for j in range(n_k)] for i in range(n_q)])
        ref = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, attn_mask=mask, scale=p["scale"])
        ref_o = ref[0].transpose(0, 1).numpy()
        s = (qh @ kh.transpose(-1, -2)) * p["scale"]
        s = s.masked_fill(~mask, float("-inf"))
        ref_lse = torch.logsumexp(s, dim=-1)[0].transpose(0, 1).numpy()
        np.testing.assert_allclose(o[qs:qs + n_q], ref_o, rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(lse[qs:qs + n_q], ref_lse, rtol=1e-10, atol=1e-10)


MIXED = [(1, 17, 16), (5, 40, 35), (3, 3, 0), (1, 64, 63), (7, 50, 20), (0, 0, 0)]


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (4, 1), (6, 3)])
def test_paged_attention_matches_sdpa(hq, hkv):
    _sdpa_check(_random_problem(7 + hq + hkv, hq, hkv, 16, MIXED))


def test_paged_attention_non_causal_matches_sdpa():
    _sdpa_check(_random_problem(3, 4, 2, 8, [(2, 20, 0), (1, 33, 32)]), causal=False)


def test_paged_attention_brute_force_python():
    """Scalar pure-Python loops in float64 (math.exp), tiny sizes."""
    p = _random_problem(11, 2, 1, 4, [(2, 5, 3), (1, 18, 17)])
    o, lse = paged_ref.paged_attention(**p)
    for r in range(2):
        n_q, n_k, qs, off = (int(p["q_lens"][r]), int(p["k_lens"][r]), int(p["q_starts"][r]),
                             int(p["q_pos_offsets"][r]))
        for i in range(n_q):
            for h in range(2):
                scores, vals = [], []
                for j in range(n_k):
                    if j > off + i:
                        continue
                    blk = int(p["block_table"][r][j // BS])
                    kv = h // 2
                    kvec = p["k_cache"][blk, j % BS, kv]
                    s = sum(float(p["q"][qs + i, h, x]) * float(kvec[x]) for x in range(4)) * p["scale"]
                    scores.append(s)
                    vals.append(p["v_cache"][blk, j % BS, kv])
                mx = max(scores)
                w = [math.exp(s - mx) for s in scores]
                tot = sum(w)
                ref = [sum(w[j] * float(vals[j][x]) for j in range(len(w))) / tot for x in range(4)]
                np.testing.assert_allclose(o[qs + i, h], ref, rtol=1e-12, atol=1e-12)
                assert abs(lse[qs + i, h] - (mx + math.log(tot))) < 1e-12


def test_single_visible_key_closed_form():
    p = _random_problem(5, 4, 2, 8, [(1, 1, 0)])
    o, lse = paged_ref.paged_attention(**p)
    blk = p["block_table"][0][0]
    for h in range(4):
        np.testing.assert_array_equal(o[0, h], p["v_cache"][blk, 0, h // 2])
        assert lse[0, h] == pytest.approx(float(p["q"][0, h] @ p["k_cache"][blk, 0, h // 2]) * p["scale"], abs=1e-12)


def test_equal_keys_give_mean_of_values():
    p = _random_problem(9, 2, 2, 8, [(1, 37, 36)])
    p["k_cache"][:] = p["k_cache"][0, 0]  # every key identical -> uniform softmax
    o, lse = paged_ref.paged_attention(**p)
    vs = paged_ref.gather_keys(p["v_cache"], p["block_table"][0], 37)
    np.testing.assert_allclose(o[0], vs.mean(axis=0), rtol=1e-12, atol=1e-12)
    s0 = float(p["q"][0, 0] @ p["k_cache"][0, 0, 0]) * p["scale"]
    assert lse[0, 0] == pytest.approx(s0 + math.log(37), abs=1e-10)


def test_block_permutation_invariance():
    p = _random_problem(21, 8, 2, 16, MIXED)
    o, lse = paged_ref.paged_attention(**p)
    n = p["k_cache"].shape[0]
    perm = np.random.default_rng(0).permutation(n)  # new id of old block b is perm[b]
    q = dict(p)
    q["k_cache"] = np.empty_like(p["k_cache"])
    q["v_cache"] = np.empty_like(p["v_cache"])
    q["k_cache"][perm] = p["k_cache"]
    q["v_cache"][perm] = p["v_cache"]
    q["block_table"] = perm[p["block_table"]].astype(np.int32)
    o2, lse2 = paged_ref.paged_attention(**q)
    np.testing.assert_array_equal(o, o2)
    np.testing.assert_array_equal(lse, lse2)


def test_split_keys_merge_by_lse():
    """Attention over keys [0, a) and [a, n) merged by their LSE equals the
    full result: pins lse as the natural-log normaliser."""
    n, a = 70, 32
    p = _random_problem(31, 4, 4, 16, [(1, n, n - 1)])
    o, lse = paged_ref.paged_attention(**p)
    lo = dict(p, k_lens=np.array([a], np.int32), q_pos_offsets=np.array([a - 1], np.int32))
    o1, l1 = paged_ref.paged_attention(**lo)
    # second half: shift the table by a/16 blocks
    hi = dict(p, k_lens=np.array([n - a], np.int32), q_pos_offsets=np.array([n - a - 1], np.int32),
              block_table=p["block_table"][:, a // BS:])
    o2, l2 = paged_ref.paged_attention(**hi)
    m = np.maximum(l1, l2)
    w1, w2 = np.exp(l1 - m), np.exp(l2 - m)
    merged = (o1 * w1[..., None] + o2 * w2[..., None]) / (w1 + w2)[..., None]
    np.testing.assert_allclose(merged, o, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(m + np.log(w1 + w2), lse, rtol=1e-12, atol=1e-12)


def test_shared_prefix_equals_duplicated_blocks():
    p = _random_problem(41, 4, 2, 8, [(1, 40, 39), (1, 50, 49)], pool=12)
    bt = p["block_table"].copy()
    bt[1, :2] = bt[0, :2]  # row 1 shares row 0's first two blocks
    shared = dict(p, block_table=bt)
    o, _ = paged_ref.paged_attention(**shared)
    dup = dict(p)
    dup["k_cache"] = p["k_cache"].copy()
    dup["v_cache"] = p["v_cache"].copy()
    for j in range(2):
        dup["k_cache"][p["block_table"][1, j]] = p["k_cache"][bt[0, j]]
        dup["v_cache"][p["block_table"][1, j]] = p["v_cache"][bt[0, j]]
    o2, _ = paged_ref.paged_attention(**dup)
    np.testing.assert_array_equal(o, o2)


MUTATIONS = {
    "gqa_map_mod_instead_of_div": ("np.repeat(k, g, axis=1)", "np.tile(k, (1, g, 1))"),
    "causal_off_by_one": (">= np.arange(n_k)", "> np.arange(n_k)"),
    "missing_scale": (") * scale", ")"),
    "lse_log2": ("np.log(np.where(lsum", "np.log2(np.where(lsum"),
    "query_offset_ignored": ("(off + np.arange(n_q))", "(np.arange(n_q))"),
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_oracle_mistakes_are_caught(name):
    src = inspect.getsource(paged_ref.paged_attention)
    old, new = MUTATIONS[name]
    assert old in src, f"mutation anchor {old!r} not found"
    ns = dict(paged_ref.__dict__)
    exec(compile(src.replace(old, new, 1), "<mutant>", "exec"), ns)
    mutant = ns["paged_attention"]
    p = _random_problem(99, 8, 2, 16, MIXED)
    with pytest.raises(AssertionError):
        _sdpa_check(p, fn=mutant)
    _sdpa_check(p)  # the real oracle passes the same check


def test_reshape_and_cache_matches_index_copy():
    rng = np.random.default_rng(1)
    n, hkv, d, s = 10, 3, 8, 13
    kc = rng.standard_normal((n, BS, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((n, BS, hkv, d)).astype(np.float32)
    key = rng.standard_normal((s, hkv, d)).astype(np.float32)
    val = rng.standard_normal((s, hkv, d)).astype(np.float32)
    slots = rng.choice(n * BS, size=s, replace=False)
    k2, v2 = paged_ref.reshape_and_cache(kc, vc, key, val, slots)
    kt, vt = torch.tensor(kc), torch.tensor(vc)
    kt.view(-1, hkv, d).index_copy_(0, torch.tensor(slots), torch.tensor(key))
    vt.view(-1, hkv, d).index_copy_(0, torch.tensor(slots), torch.tensor(val))
    np.testing.assert_array_equal(k2, kt.numpy())
    np.testing.assert_array_equal(v2, vt.numpy())
    # padding slots are skipped, the rest still lands
    slots_pad = slots.copy()
    slots_pad[0] = -1
    k3, _ = paged_ref.reshape_and_cache(kc, vc, key, val, slots_pad)
    np.testing.assert_array_equal(k3.reshape(-1, hkv, d)[slots[1:]], key[1:])
    assert np.array_equal(k3.reshape(-1, hkv, d)[slots[0]], kc.reshape(-1, hkv, d)[slots[0]])


def test_copy_blocks_brute_force():
    rng = np.random.default_rng(2)
    kv = rng.integers(0, 2**16, size=(3, 2, 9, 4, 2, 8), dtype=np.uint16)
    src, dst = np.array([1, 4, 4]), np.array([0, 7, 8])
    out = paged_ref.copy_blocks(kv, src, dst)
    for layer in range(3):
        for kvi in range(2):
            for b in range(9):
                exp = kv[layer, kvi, src[list(dst).index(b)]] if b in dst else kv[layer, kvi, b]
                np.testing.assert_array_equal(out[layer, kvi, b], exp)


class _Phase:
    def __init__(self, name):
        self.name = name


class _Req:
    def __init__(self, rid, phase, computed, total, bt):
        self.request_id, self.phase = rid, _Phase(phase)
        self.num_computed_tokens, self.total_len, self.block_table = computed, total, bt


def _known_answer_step():
    reqs = [
        _Req("a", "NEEDS_PREFILL", 14, 18, [7, 3]),
        _Req("b", "NEEDS_DECODE", 32, 33, [5, 9, 2]),
        _Req("c", "NEEDS_PREFILL", 16, 16, [1]),  # fully prefix-matched: 0-token chunk
    ]
    return reqs, {"a": 4, "c": 0}


def test_metadata_known_answer():
    reqs, chunks = _known_answer_step()
    rows = paged_ref.step_rows(reqs, chunks)
    q_lens, k_lens, q_starts, offs, bt, mb, total = paged_ref.batch_metadata(rows)
    assert q_lens.tolist() == [4, 1, 0]
    assert k_lens.tolist() == [18, 33, 16]
    assert q_starts.tolist() == [0, 4, 5]
    assert offs.tolist() == [14, 32, 16]
    assert bt.tolist() == [[7, 3, 0], [5, 9, 2], [1, 0, 0]]
    assert (mb, total) == (3, 5)
    slots, pos = paged_ref.write_slots_and_positions(rows, BS)
    assert slots.tolist() == [126, 127, 48, 49, 32]
    assert pos.tolist() == [14, 15, 16, 17, 32]


def test_eager_restatement_matches_oracle_fp32():
    """The torch eager path (fp32) agrees with the fp64 oracle, whole-batch and per-row."""
    p = _random_problem(55, 8, 2, 32, [(1, 17, 16), (6, 40, 34), (1, 64, 63)])
    rows = [(int(a), int(b), int(c), p["block_table"][i]) for i, (a, b, c) in
            enumerate(zip(p["q_lens"], p["k_lens"], p["q_pos_offsets"]))]
    t = int(p["q_lens"].sum())
    # the step appends each query's own K/V first
    slots, _ = paged_ref.write_slots_and_positions(rows, BS)
    rng = np.random.default_rng(3)
    kn = rng.standard_normal((t, 2, 32))
    vn = rng.standard_normal((t, 2, 32))
    kc, vc = paged_ref.reshape_and_cache(p["k_cache"], p["v_cache"], kn, vn, slots)
    o_ref, _ = paged_ref.paged_attention(**dict(p, k_cache=kc, v_cache=vc))
    outs = []
    for per_row in (False, True):
        o = eager.eager_step(torch.tensor(p["q"], dtype=torch.float32),
                             torch.tensor(kn, dtype=torch.float32), torch.tensor(vn, dtype=torch.float32),
                             torch.tensor(p["k_cache"], dtype=torch.float32),
                             torch.tensor(p["v_cache"], dtype=torch.float32),
                             torch.tensor(slots), rows, p["scale"], 2, per_row=per_row)
        np.testing.assert_allclose(o.numpy(), o_ref, rtol=1e-5, atol=1e-5)
        outs.append(o)
    torch.testing.assert_close(outs[0], outs[1], rtol=1e-6, atol=1e-6)
