"""CPU checks of the C ABI: libkvhot.so loads, exports exactly what
include/kvhot.h declares, and its host-side validation rejects bad arguments
before touching a GPU (no kernel is launched by these tests)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, sea_module

HEADER = os.path.join(ROOT, "include", "kvhot.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvhot_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return sea_module("_lib").load()


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) == 8
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(sea_module("_lib").SIGNATURES) == names


def test_version_and_error_string(lib):
    assert lib.kvhot_version() == 100
    assert isinstance(lib.kvhot_last_error(), bytes)


# Fake, 16-byte aligned device addresses: every call below must return before
# any launch, and these tests never run where a GPU is visible.
FAKE = 1 << 20
no_gpu = pytest.mark.skipif(__import__("torch").cuda.is_available(),
                            reason="passes fake device pointers; CPU-only check")


def _i64(*v):
    return (ctypes.c_int64 * len(v))(*v)


@no_gpu
def test_reshape_and_cache_rejects_bad_arguments(lib):
    st3, st4 = _i64(1024, 128, 1), _i64(16384, 1024, 128, 1)
    # bad dtype
    assert lib.kvhot_reshape_and_cache(1, st3, 1, st3, 1, st4, 1, st4, 1, 1, 4, 8, 128, 16, 10, 9, None) == -1
    assert b"dtype" in lib.kvhot_last_error()
    # head_dim not unit-stride
    assert lib.kvhot_reshape_and_cache(1, _i64(1024, 128, 2), 1, st3, 1, st4, 1, st4, 1, 1, 4, 8, 128,
                                       16, 10, 2, None) == -1
    # zero tokens is a no-op success
    assert lib.kvhot_reshape_and_cache(None, st3, None, st3, None, st4, None, st4, None, 1, 0, 8, 128,
                                       16, 10, 2, None) == 0


@no_gpu
def test_copy_blocks_rejects_bad_arguments(lib):
    assert lib.kvhot_copy_blocks(1, 0, 0, 0, 0, 64, 10, 1, 1, 1, None) == -1
    assert lib.kvhot_copy_blocks(None, 1, 0, 0, 0, 64, 10, 1, 1, 1, None) == -1
    assert lib.kvhot_copy_blocks(None, 1, 0, 0, 0, 64, 10, None, None, 0, None) == 0


@no_gpu
def test_attention_rejects_bad_arguments(lib):
    q3, c4, l2 = _i64(4096, 128, 1), _i64(16384, 1024, 128, 1), _i64(32, 1)
    f = FAKE
    args = [f, q3, f, c4, f, c4, f, q3, f, l2, f, 8, f, f, f, f,
            4, 4, 1, 100, 32, 8, 128, 16, 64, 0.1, 1, 2, 64, None, None, None, 0, None]
    bad = list(args)
    bad[20] = 30  # Hq not a multiple of Hkv
    assert lib.kvhot_paged_attention(*bad) == -1
    bad = list(args)
    bad[27] = 5  # dtype
    assert lib.kvhot_paged_attention(*bad) == -1
    bad = list(args)
    bad[28] = 48  # partition not a multiple of 32
    assert lib.kvhot_paged_attention(*bad) == -1
    assert b"partition" in lib.kvhot_last_error()
    bad = list(args)
    bad[1] = _i64(4096, 128, 2)  # head_dim stride
    assert lib.kvhot_paged_attention(*bad) == -1
    # split-K plan needs a workspace: none given -> KVHOT_EWORKSPACE (-3), before any launch
    assert lib.kvhot_paged_attention(*args) == -3
    assert b"workspace" in lib.kvhot_last_error()
    # empty batch is a successful no-op
    empty = list(args)
    empty[16] = 0
    assert lib.kvhot_paged_attention(*empty) == 0


@no_gpu
def test_attention_checks_the_schedule_description(lib):
    """A schedule comes with its description; the description must add up,
    and the workspace must hold what it asks for (checked before any launch)."""
    q3, c4, l2 = _i64(4096, 128, 1), _i64(16384, 1024, 128, 1), _i64(32, 1)
    f = FAKE
    info = _i64(7, 0, 7, 2, 1000 + 16384, 1, 4096, 8)  # 7 decode units, 2 work-groups, 17384 workspace bytes
    args = [f, q3, f, c4, f, c4, f, q3, f, l2, f, 8, f, f, f, f,
            4, 4, 1, 100, 32, 8, 128, 16, 64, 0.1, 1, 2, 0, f, info, None, 0, None]
    bad = list(args)
    bad[30] = None  # schedule without its description
    assert lib.kvhot_paged_attention(*bad) == -1
    assert b"schedule_info" in lib.kvhot_last_error()
    bad = list(args)
    bad[30] = _i64(9, 0, 7, 2, 0, 0, 4096, 8)  # unit counts do not add up
    assert lib.kvhot_paged_attention(*bad) == -1
    bad[30] = _i64(7, 0, 7, 2, 0, 0, 4096, 3)  # no such bank count
    assert lib.kvhot_paged_attention(*bad) == -1
    # the description asks for 17384 workspace bytes: none, or fewer, is KVHOT_EWORKSPACE
    assert lib.kvhot_paged_attention(*args) == -3
    short = list(args)
    short[31], short[32] = f, 17383
    assert lib.kvhot_paged_attention(*short) == -3
    assert b"17384" in lib.kvhot_last_error()


def test_workspace_bytes(lib):
    # decode: 64 rows, max ctx 2048, 32/8 heads, D=128, 256-token partitions
    # -> counter bytes, then 64 rows x 8 kv heads x 8 parts partials of 4 heads x (128 + 1) floats
    n = lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 32, 8, 128, 16, 256, 2)
    assert n == 16384 + 64 * 8 * 8 * 4 * (128 + 1) * 4
    assert sea_module("_lib").WORKSPACE_COUNTER_BYTES == 16384
    # one partition: no workspace
    assert lib.kvhot_paged_attention_workspace_bytes(4, 4, 1, 130, 12, 12, 64, 16, 512, 2) == 0
    # fp32 runs the VALU kernel, which never splits
    assert lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 32, 8, 128, 16, 256, 0) == 0
    assert lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 30, 8, 128, 16, 256, 2) < 0


def _schedule(lib, q_lens, k_lens, offs, hq=32, hkv=8, d=128, pt=0, causal=1, dtype=2):
    """Runs the host planner; returns (decode section as a dict, prefill
    units, info, query token of each row)."""
    import numpy as np

    q = np.asarray(q_lens, np.int32)
    k = np.asarray(k_lens, np.int32)
    o = np.asarray(offs, np.int32)
    qs = np.concatenate([[0], np.cumsum(q)[:-1]]).astype(np.int32)
    info = (ctypes.c_int64 * 8)()
    head = (q.ctypes.data, k.ctypes.data, qs.ctypes.data, o.ctypes.data, len(q), hq, hkv, d, 16, pt, causal,
            dtype)
    total = lib.kvhot_paged_attention_schedule(*head, None, 0, info)
    units = np.zeros((max(total, 0), 8), np.int32)
    got = lib.kvhot_paged_attention_schedule(*head, units.ctypes.data, total, info)
    assert got == total == info[0]
    npre, ndec, groups, ws, cut_rows = info[1], info[2], info[3], info[4], info[5]
    assert npre + ndec == total
    pre = units[:npre]
    dec = None
    if ndec:
        sec = units[npre:]
        nwg, npc, nemp, maxs, maxp = sec[0, :5]
        assert nwg == groups and 1 + nwg + 2 * npc + nemp == ndec
        hdr = sec[1:1 + nwg]
        pcs = sec[1 + nwg:1 + nwg + 2 * npc].reshape(npc, 16)  # two units per piece
        emp = sec[1 + nwg + 2 * npc:]
        assert (pcs[:, 9:] == 0).all()
        assert max(h[2] for h in hdr.tolist()) == maxs <= 4096 and max(h[1] for h in hdr.tolist()) == maxp <= 256
        dec = dict(hdr=hdr, pieces=pcs, empties=emp[:, 0].tolist(), ws=ws, cut_rows=cut_rows)
        assert 0 < info[6] <= 160 * 1024 and info[7] & 255 in (4, 8) and info[7] >> 9 == 0
    return dec, pre, info, qs


def _check_decode_schedule(dec, kends, qs, hkv, G=4, D=128, pt=0):
    """Head groups: work-group g reads kv head (g + g // hkv) % hkv of group g // hkv, and
    a group's work-groups share one piece list; every decode row's slices are
    covered exactly once per kv head by pieces in row order; a work-group
    lists its cut rows first; a cut row's pieces are numbered along the row
    and have their own counter and row partials; rows with no visible key are
    listed as empty.  Returns the slices of each group."""
    hdr, pcs = dec["hdr"], dec["pieces"]
    groups = {}
    cover = {}
    cut_of, prow_of = {}, {}
    for g, (poff, pcnt, slices, kvh, grp, *_rest) in enumerate(hdr.tolist()):
        assert kvh == (g % hkv + g // hkv) % hkv and grp == g // hkv  # heads rotate with the group
        if grp in groups:
            assert groups[grp][:2] == (poff, pcnt)
        mine = pcs[poff:poff + pcnt].tolist()
        assert sum(p[2] - p[1] for p in mine) == slices
        groups[grp] = (poff, pcnt, slices)
        seen_whole = False
        first_want = 0
        for row, s0, s1, npi, qtok, kend, cut, prow, first, *_ in mine:
            assert first == first_want  # the piece's first slice in the work-group's order
            first_want += s1 - s0
            np_, idx = npi & 0xFFFF, npi >> 16
            assert s0 < s1 and qtok == qs[row] and kend == kends[row]
            if np_ > 1:
                assert not seen_whole, "cut pieces come first"
                assert cut_of.setdefault(row, cut) == cut and prow_of.setdefault(row, prow) == prow
                assert 0 <= idx < np_
                if pt:
                    assert s0 % (pt // 16) == 0 or s0 == 0
            else:
                seen_whole = True
                assert (s0, s1, cut) == (0, -(-kends[row] // 16), -1)
            cover.setdefault((row, kvh), []).append((s0, s1, idx, np_))
    for row, kend in kends.items():
        n = -(-kend // 16)
        for h in range(hkv):
            if n == 0:
                assert (row, h) not in cover
                continue
            ps = sorted(cover.pop((row, h)))
            assert ps[0][0] == 0 and ps[-1][1] == n
            assert all(x[1] == y[0] for x, y in zip(ps, ps[1:]))
            assert [x[2] for x in ps] == list(range(len(ps))) and all(x[3] == len(ps) for x in ps)
    assert not cover
    assert sorted(dec["empties"]) == sorted(int(qs[r]) for r, k in kends.items() if k == 0)
    # counters and row partials of the cut rows are disjoint
    assert sorted(cut_of.values()) == list(range(len(cut_of))) == list(range(dec["cut_rows"]))
    pieces_of = {r: sum(1 for p in pcs.tolist() if p[0] == r) for r in cut_of}
    spans = sorted((prow_of[r], prow_of[r] + pieces_of[r]) for r in cut_of)
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    nrp = sum(e - s for s, e in spans)
    assert dec["ws"] == (16384 + nrp * hkv * G * (D + 1) * 4 if cut_of else 0)
    return [groups[q][2] for q in sorted(groups)]


def test_schedule_lists_every_unit_once(lib):
    """Host planner: decode pieces cover every (row, kv head) once; prefill
    units every (row, kv head, query block), longest first."""
    # rows: decode 300 keys, decode 40 keys, prefill 20 queries on 50 keys, empty chunk, decode 2000 keys
    q_lens, k_lens, offs = [1, 1, 20, 0, 1], [300, 40, 50, 16, 2000], [299, 39, 30, 16, 1999]
    dec, pre, info, qs = _schedule(lib, q_lens, k_lens, offs, pt=1024)
    _check_decode_schedule(dec, {0: 300, 1: 40, 4: 2000}, qs, 8, pt=1024)
    # prefill: 20 queries, 64 per work-group (8 waves x 32 m-rows / G=4) -> 1 block x 8 kv heads;
    # the empty chunk has none
    assert sorted(map(tuple, pre[:, :3].tolist())) == sorted((2, h, 0) for h in range(8))
    # the block's last query (position 49) sees 50 keys: two 32-key tiles
    assert sorted(set(pre[:, 3].tolist())) == [2]
    assert list(pre[:, 3]) == sorted(pre[:, 3], reverse=True)


def test_schedule_prefill_blocks_longest_first(lib):
    """Prefill work-groups take 64 queries (G=4) and are listed by key tiles, most first."""
    # one 150-query chunk at positions 100..249 (250 keys), one 40-query chunk on 40 keys
    dec, pre, info, qs = _schedule(lib, [150, 40], [250, 40], [100, 0])
    assert dec is None and info[4] == 0
    units = sorted(map(tuple, pre[:, :4].tolist()))
    # row 0: blocks of queries 0-63, 64-127, 128-149 -> visible keys 164, 228, 250 -> 6, 8, 8 tiles
    want = [(0, h, b, t) for h in range(8) for b, t in ((0, 6), (1, 8), (2, 8))]
    want += [(1, h, 0, 2) for h in range(8)]
    assert units == sorted(want)
    assert list(pre[:, 3]) == sorted(pre[:, 3], reverse=True)


def test_schedule_head_groups_balance_the_gqa_batch(lib):
    """The 64-row GQA decode shape: 32 groups of 8 work-groups (256 when no
    device is queried), every group within a few slices of the even cut, at
    most one row cut at each end of a range."""
    import numpy as np

    rng = np.random.default_rng(0)
    ctx = rng.integers(128, 2048, size=64, endpoint=True)
    dec, pre, info, qs = _schedule(lib, [1] * 64, ctx, ctx - 1)
    assert len(pre) == 0 and info[3] == 256
    loads = _check_decode_schedule(dec, dict(enumerate(ctx.tolist())), qs, 8)
    total = sum(-(-int(c) // 16) for c in ctx)
    target = -(-total // 32)
    assert len(loads) == 32 and sum(loads) == total
    assert max(loads) <= target + 4 and min(loads[:-1]) >= target - 4
    cuts_per_group = [sum(1 for p in dec["pieces"][h[0]:h[0] + h[1]].tolist() if p[3] & 0xFFFF > 1)
                      for h in dec["hdr"][::8].tolist()]
    assert max(cuts_per_group) <= 2 and 0 < dec["cut_rows"] <= 31


def test_schedule_cuts_long_rows_on_partitions(lib):
    """16 rows of 32768 keys (the long-context shape): two groups per row,
    cuts on 512-key partition boundaries."""
    ctx = [32768] * 16
    dec, pre, info, qs = _schedule(lib, [1] * 16, ctx, [c - 1 for c in ctx], pt=512)
    loads = _check_decode_schedule(dec, dict(enumerate(ctx)), qs, 8, pt=512)
    assert loads == [1024] * 32 and dec["cut_rows"] == 16
    assert info[4] == 16384 + 16 * 2 * 8 * 4 * 129 * 4


def test_schedule_tiny_rows_and_empty_rows(lib):
    """Rows with no visible key are listed for zero output; tiny rows are
    never cut below 4 slices."""
    q_lens = [1] * 40
    k_lens = [0, 5] + [17] * 38
    offs = [0, 4] + [16] * 38
    dec, pre, info, qs = _schedule(lib, q_lens, k_lens, offs, hq=8, hkv=8, d=64)
    kends = dict(enumerate(min(k, o + 1) for k, o in zip(k_lens, offs)))
    _check_decode_schedule(dec, kends, qs, 8, G=1, D=64)
    assert dec["empties"] == [0]
    assert dec["cut_rows"] == 0 and info[4] == 0


def test_schedule_empty_for_vector_path(lib):
    # fp32 runs the VALU kernel: no launch list
    dec, pre, info, _ = _schedule(lib, [1, 1], [100, 50], [99, 49], dtype=0)
    assert dec is None and len(pre) == 0 and info[4] == 0 and info[0] == 0
