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
    assert len(names) == 9
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
            4, 4, 1, 100, 32, 8, 128, 16, 64, 0.1, 1, 2, 64, None, 0, 0, 0, 0, 0, None, 0, None]
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
    bad = list(args)
    bad[26] = 8  # attn_flags: only KVHOT_CAUSAL (1), KVHOT_DETERMINISTIC (2) and KVHOT_VERIFY_BLOCKS (4) exist
    assert lib.kvhot_paged_attention(*bad) == -1
    assert b"attn_flags" in lib.kvhot_last_error()
    det = list(args)
    det[26] = 3  # causal + deterministic: valid, so it gets as far as the workspace check
    assert lib.kvhot_paged_attention(*det) == -3
    # split-K plan needs a workspace: none given -> KVHOT_EWORKSPACE (-3), before any launch
    assert lib.kvhot_paged_attention(*args) == -3
    assert b"workspace" in lib.kvhot_last_error()
    # empty batch is a successful no-op
    empty = list(args)
    empty[16] = 0
    assert lib.kvhot_paged_attention(*empty) == 0


@no_gpu
def test_attention_checks_the_schedule_workspace(lib):
    """A schedule's reported workspace size comes with it: a workspace
    shorter than that is KVHOT_EWORKSPACE before any launch, and a schedule
    with merge or shared-prefix units must report room for its partials."""
    q3, c4, l2 = _i64(4096, 128, 1), _i64(16384, 1024, 128, 1), _i64(32, 1)
    f = FAKE
    need = 10 * 4 * (128 + 1) * 4  # 10 partials of 4 query heads x (128 + 1) floats
    # two 8-wave decode work-groups and one merge unit
    args = [f, q3, f, c4, f, c4, f, q3, f, l2, f, 8, f, f, f, f,
            4, 4, 1, 100, 32, 8, 128, 16, 64, 0.1, 1, 2, 0, f, 16, 0, 1, 0, need, f, need - 1, None]
    assert lib.kvhot_paged_attention(*args) == -3
    assert str(need).encode() in lib.kvhot_last_error()
    bad = list(args)
    bad[34] = 100  # less than one partial
    assert lib.kvhot_paged_attention(*bad) == -1
    bad[34] = -1
    assert lib.kvhot_paged_attention(*bad) == -1
    # shared-prefix units are counted among the prefill units, and need partials too
    pfx = list(args)
    pfx[31:35] = [2, 0, 3, need]  # more prefix units than prefill units
    assert lib.kvhot_paged_attention(*pfx) == -1
    pfx[31:35] = [2, 0, 2, 100]
    assert lib.kvhot_paged_attention(*pfx) == -1
    pfx[31:35] = [2, 0, -1, need]
    assert lib.kvhot_paged_attention(*pfx) == -1


@no_gpu
def test_noalloc_rejects_calls_beyond_its_scratch(lib):
    """The no-alloc variant holds at most 64 MiB of split-K partials; a call
    that needs more is KVHOT_EWORKSPACE before it touches a device."""
    assert sea_module("_lib").NOALLOC_SCRATCH_BYTES == 64 << 20
    q3, c4, l2 = _i64(4096, 128, 1), _i64(16384, 1024, 128, 1), _i64(32, 1)
    f = FAKE
    # no schedule: 64 rows of up to 65536 keys in 32-key partitions -> 64 x 8 x 2048 partials of 2064 bytes
    args = [f, q3, f, c4, f, c4, f, q3, f, l2, f, 4096, f, f, f, f,
            64, 64, 1, 65536, 32, 8, 128, 16, 1 << 20, 0.1, 1, 2, 32, None, 0, 0, 0, 0, 0, None]
    assert lib.kvhot_paged_attention_noalloc(*args) == -3
    msg = lib.kvhot_last_error()
    assert str(64 * 8 * 2048 * 4 * 129 * 4).encode() in msg and b"67108864" in msg
    # a schedule whose merge units need one byte more than the scratch
    sched = list(args)
    sched[29:35] = [f, 16, 0, 1, 0, (64 << 20) + 1]
    assert lib.kvhot_paged_attention_noalloc(*sched) == -3
    # shared-prefix units alone (no merge units) need their partials too
    sched[29:35] = [f, 16, 2, 0, 2, (64 << 20) + 1]
    assert lib.kvhot_paged_attention_noalloc(*sched) == -3
    # invalid sizes are reported as such
    bad = list(args)
    bad[20] = 30
    assert lib.kvhot_paged_attention_noalloc(*bad) == -1


def test_workspace_bytes(lib):
    # decode: 64 rows, max ctx 2048, 32/8 heads, D=128, 256-token partitions
    # -> 64 rows x 8 kv heads x 8 parts partials of 4 heads x (128 + 1) floats
    n = lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 32, 8, 128, 16, 256, 2)
    assert n == 64 * 8 * 8 * 4 * (128 + 1) * 4
    # one partition: no workspace
    assert lib.kvhot_paged_attention_workspace_bytes(4, 4, 1, 130, 12, 12, 64, 16, 512, 2) == 0
    # fp32 runs the VALU kernel, which never splits
    assert lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 32, 8, 128, 16, 256, 0) == 0
    assert lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 30, 8, 128, 16, 256, 2) < 0


# Waves per decode work-group, and decode work-groups of a device-full where
# no device is visible (one on each of 256 CUs).
W = 8
GROUPS = 256


def _schedule(lib, q_lens, k_lens, offs, hq=32, hkv=8, d=128, pt=0, causal=1, dtype=2, bt=None,
              prefix=False):
    """Runs the host planner; returns (decode descriptors as dicts, prefill
    units, merge units, workspace bytes, query token of each row), and with
    prefix=True also the number of shared-prefix units (the first ones of
    the prefill units).  Without `bt`, row r's block j is 1000 + r*mb + j
    (no blocks shared)."""
    import numpy as np

    q = np.asarray(q_lens, np.int32)
    k = np.asarray(k_lens, np.int32)
    o = np.asarray(offs, np.int32)
    qs = np.concatenate([[0], np.cumsum(q)[:-1]]).astype(np.int32)
    if bt is None:
        mb = max(-(-int(x) // 16) for x in k)
        bt = (np.arange(len(q) * mb, dtype=np.int32).reshape(len(q), mb) + 1000)
    bt = np.ascontiguousarray(bt, np.int32)
    mb = bt.shape[1]
    cnt = [ctypes.c_int64() for _ in range(5)]
    outs = tuple(ctypes.byref(c) for c in cnt)
    head = (q.ctypes.data, k.ctypes.data, qs.ctypes.data, o.ctypes.data, bt.ctypes.data, mb, len(q), hq, hkv,
            d, 16, pt, causal, dtype)
    total = lib.kvhot_paged_attention_schedule(*head, None, 0, *outs)
    units = np.zeros((max(total, 0), 8), np.int32)
    got = lib.kvhot_paged_attention_schedule(*head, units.ctypes.data, total, *outs)
    assert got == total
    nd, npf, nm, ws, npx = (c.value for c in cnt)
    assert nd + npf + nm == total and 0 <= npx <= npf
    dec = []
    for x, y, s0, s1, qtok, kend, first, pidx in units[:nd].tolist():
        if x < 0:
            dec.append(None)
            continue
        row, nparts, kvh, part = x & 0xFFFF, x >> 16, y & 0xFFFF, (y >> 16) & 0xFFFF
        # each descriptor carries its row's query token, visible keys and first block
        assert qtok == qs[row] and kend == min(k[row], o[row] + 1)
        assert first == (bt[row, s0] if s0 < s1 else -1)
        dec.append(dict(row=row, nparts=nparts, kvh=kvh, part=part, s0=s0, s1=s1, pidx=pidx))
    if prefix:
        return dec, units[nd:nd + npf], units[nd + npf:], ws, qs, npx
    assert npx == 0
    return dec, units[nd:nd + npf], units[nd + npf:], ws, qs


def _check_decode_schedule(dec, merge, ws, qs, W, rows, hkv, G=4, D=128, pt=0):
    """Every (row, kv head) key range of every decode row is covered exactly
    once by parts; each part is one contiguous run of waves of one
    work-group; split ranges have one merge unit whose partial indices are
    theirs alone; the workspace holds every partial.  Returns the slices per
    work-group."""
    assert len(dec) % W == 0
    cover, owner, loads = {}, {}, []
    for g0 in range(0, len(dec), W):
        grp = dec[g0:g0 + W]
        load, prev = 0, None
        for wv in grp:
            if wv is None:
                prev = None
                continue
            key = (wv["row"], wv["kvh"], wv["part"])
            if key != prev:
                assert key not in owner, "part in two places"
                owner[key] = g0
            prev = key
            load += wv["s1"] - wv["s0"]
            cover.setdefault((wv["row"], wv["kvh"]), []).append(wv)
        loads.append(load)
    base_of = {}
    for qtok, kvh, nparts, base, *rest in merge.tolist():
        assert rest == [0, 0, 0, 0]
        base_of[(qtok, kvh)] = (nparts, base)
    used = set()
    for row, kend in rows.items():
        n = -(-kend // 16)
        for h in range(hkv):
            waves = sorted(cover.pop((row, h)), key=lambda w: (w["s0"], w["s1"]))
            nparts = waves[0]["nparts"]
            assert all(w["nparts"] == nparts for w in waves)
            assert waves[0]["s0"] == 0 and waves[-1]["s1"] == n
            assert all(a["s1"] == b["s0"] for a, b in zip(waves, waves[1:]))
            parts = sorted({w["part"] for w in waves})
            assert parts == list(range(nparts))
            for w in waves:
                if pt:
                    assert w["part"] * pt // 16 <= w["s0"] and w["s1"] <= (w["part"] + 1) * pt // 16
                if nparts > 1:
                    used.add(w["pidx"])
            if nparts > 1:
                nm, base = base_of.pop((int(qs[row]), h))
                assert nm == nparts
                assert {w["pidx"] for w in waves} == set(range(base, base + nparts))
                assert all(w["pidx"] == base + w["part"] for w in waves)
    assert not cover and not base_of
    assert ws == len(used) * G * (D + 1) * 4
    return loads


def test_schedule_lists_every_unit_once(lib):
    """Host planner: decode waves cover every (row, kv head, partition) once;
    prefill units every (row, kv head, query block); longest first."""
    # rows: decode 300 keys, decode 40 keys, prefill 20 queries on 50 keys, empty chunk, decode 2000 keys
    q_lens, k_lens, offs = [1, 1, 20, 0, 1], [300, 40, 50, 16, 2000], [299, 39, 30, 16, 1999]
    dec, pre, merge, ws, qs = _schedule(lib, q_lens, k_lens, offs, pt=1024)
    _check_decode_schedule(dec, merge, ws, qs, W, {0: 300, 1: 40, 4: 2000}, 8, pt=1024)
    # the 2000-key row has two 1024-key partitions per kv head, the others one
    assert sorted(merge[:, 2].tolist()) == [2] * 8
    # prefill: 20 queries, 32 per work-group at head_dim 128 (4 waves x 32 m-rows / G=4) -> 1 block x 8 kv heads;
    # the empty chunk has none
    assert sorted(map(tuple, pre[:, :3].tolist())) == sorted((2, h, 0) for h in range(8))
    # the block's last query (position 49) sees 50 keys: two 32-key tiles
    assert sorted(set(pre[:, 3].tolist())) == [2]
    assert list(pre[:, 3]) == sorted(pre[:, 3], reverse=True)


def test_schedule_prefill_blocks_longest_first(lib):
    """Prefill work-groups take 32 queries at head_dim 128 (4 waves x 32
    m-rows / G=4) and are listed by key tiles, most first."""
    # one 150-query chunk at positions 100..249 (250 keys), one 40-query chunk on 40 keys
    dec, pre, merge, ws, qs = _schedule(lib, [150, 40], [250, 40], [100, 0])
    assert len(dec) == 0 and len(merge) == 0
    units = sorted(map(tuple, pre[:, :4].tolist()))
    # row 0: blocks of queries 0-31, ..., 128-149 -> visible keys 132, 164, 196, 228, 250 -> 5, 6, 7, 8, 8 tiles
    want = [(0, h, b, t) for h in range(8) for b, t in ((0, 5), (1, 6), (2, 7), (3, 8), (4, 8))]
    # row 1: queries 0-31 see 32 keys (1 tile), 32-39 see 40 (2 tiles)
    want += [(1, h, b, t) for h in range(8) for b, t in ((0, 1), (1, 2))]
    assert units == sorted(want)
    assert list(pre[:, 3]) == sorted(pre[:, 3], reverse=True)


def test_schedule_uncut_when_balanced(lib):
    """Many rows of mixed lengths (the 64-row GQA decode shape): whole
    (row, kv head) segments packed longest first fit one device-full (256
    work-groups of 8 waves when no device is queried) within a merge
    launch's worth of slices of the even cut, so no segment is cut and there
    is no merge launch."""
    import numpy as np

    rng = np.random.default_rng(0)
    ctx = rng.integers(128, 2048, size=64, endpoint=True)
    dec, pre, merge, ws, qs = _schedule(lib, [1] * 64, ctx, ctx - 1)
    assert len(pre) == 0
    loads = _check_decode_schedule(dec, merge, ws, qs, W, dict(enumerate(ctx.tolist())), 8)
    total = sum(-(-int(c) // 16) for c in ctx) * 8
    target = -(-total // 256)
    assert len(merge) == 0 and ws == 0
    assert len(loads) <= 256
    # 5 us of merge launch at 8 KiB slices and 5.5 TB/s over 256 work-groups: 13 slices
    assert max(loads) <= target + 13


def test_schedule_uncut_mixes_kv_heads(lib):
    """Whole-segment packing spreads each row's kv heads over work-groups so
    that every work-group holds several heads (kv heads stream at different
    rates, and a work-group of one head would end with its head's rate): 256
    rows of about 1000 tokens give every work-group all 8 heads, 64 rows of
    128-2048 tokens two heads per work-group, with the same load bound."""
    import numpy as np

    rng = np.random.default_rng(1)
    for lo, hi, rows, want in ((1000, 1100, 256, 8), (128, 2048, 64, 2)):
        ctx = rng.integers(lo, hi, size=rows, endpoint=True)
        dec, pre, merge, ws, qs = _schedule(lib, [1] * rows, ctx, ctx - 1)
        loads = _check_decode_schedule(dec, merge, ws, qs, W, dict(enumerate(ctx.tolist())), 8)
        assert len(merge) == 0
        total = sum(-(-int(c) // 16) for c in ctx) * 8
        assert max(loads) <= -(-total // 256) + 13
        heads = [len({w["kvh"] for w in dec[g:g + W] if w}) for g in range(0, len(dec), W)]
        assert min(heads) >= want, (rows, sorted(set(heads)))


def test_schedule_cuts_long_rows(lib):
    """A few long rows cannot fill the device whole: segments are cut into
    parts of equal work-group loads, joined by merge units, and every cut
    leaves at least 4 slices on either side."""
    ctx = [32768] * 4 + [1000, 3000]
    dec, pre, merge, ws, qs = _schedule(lib, [1] * len(ctx), ctx, [c - 1 for c in ctx])
    loads = _check_decode_schedule(dec, merge, ws, qs, W, dict(enumerate(ctx)), 8)
    total = sum(-(-c // 16) for c in ctx) * 8
    target = -(-total // 256)
    assert len(merge) > 0 and ws > 0
    assert len(loads) <= 257
    assert max(loads) <= target + max(2, target // 32)


def test_schedule_tiny_rows_and_empty_rows(lib):
    """Rows with no visible key still get a wave (it writes zeros); many tiny
    rows are packed at most 8 ranges per work-group, unsplit."""
    q_lens = [1] * 40
    k_lens = [0, 5] + [17] * 38
    offs = [0, 4] + [16] * 38
    dec, pre, merge, ws, qs = _schedule(lib, q_lens, k_lens, offs, hq=8, hkv=8, d=64)
    _check_decode_schedule(dec, merge, ws, qs, W, dict(enumerate(min(k, o + 1) for k, o in zip(k_lens, offs))),
                           8, G=1, D=64)
    assert len(merge) == 0 and ws == 0


def test_schedule_limits_partitions_per_row(lib):
    """A decode row's partition count is packed into 15 bits of its wave
    descriptors: 32767 partitions are scheduled, 32768 leave the call without
    a schedule (the grid path takes it)."""
    import numpy as np

    for parts, scheduled in ((32767, True), (32768, False)):
        k = np.array([32 * parts], np.int32)
        q = np.array([1], np.int32)
        o = k - 1
        qs = np.zeros(1, np.int32)
        mb = -(-int(k[0]) // 16)
        bt = np.arange(mb, dtype=np.int32).reshape(1, mb)
        cnt = [ctypes.c_int64() for _ in range(5)]
        total = lib.kvhot_paged_attention_schedule(
            q.ctypes.data, k.ctypes.data, qs.ctypes.data, o.ctypes.data, bt.ctypes.data, mb, 1, 32, 8, 128,
            16, 32, 1, 2, None, 0, *(ctypes.byref(c) for c in cnt))
        assert (total > 0) == scheduled, (parts, total)
        if scheduled:
            assert cnt[2].value == 8  # one merge unit per kv head
            assert cnt[3].value == 8 * parts * 4 * (128 + 1) * 4


def test_schedule_empty_for_vector_path(lib):
    # fp32 runs the VALU kernel: no launch list
    dec, pre, merge, ws, _ = _schedule(lib, [1, 1], [100, 50], [99, 49], dtype=0)
    assert len(dec) == 0 and len(pre) == 0 and len(merge) == 0 and ws == 0


FOLD = 0x8000  # part field of a decode segment that folds in shared-prefix partials


def _shared_prefix_segments(dec, merge, qs, rows, k_lens, hkv, shared_blocks, ks):
    """Checks the decode segments of a schedule with shared prefixes and
    returns {(row, kv head): first prefix partial} for the rows in `rows`
    (those that share `shared_blocks` blocks).  Such a segment covers the
    row's tail only.  Left whole, it folds the prefix partials itself
    (part FOLD, parts field ks, partial index = first prefix partial); cut,
    its parts are ordinary parts and its merge unit names the prefix
    partials as its extra inputs (first, ks).  Other rows start at key 0."""
    units = {}
    for qtok, kvh, n, b, xb, xn, z0, z1 in merge.tolist():
        assert z0 == 0 and z1 == 0
        units[(qtok, kvh)] = (n, b, xb, xn)
    segs = {}
    for g0 in range(0, len(dec), W):
        for wv in dec[g0:g0 + W]:
            if wv is not None:
                segs.setdefault((wv["row"], wv["kvh"]), []).append((g0, wv))
    pidx_of, cut = {}, 0
    for (row, h), waves in segs.items():
        waves.sort(key=lambda t: t[1]["s0"])
        n = -(-k_lens[row] // 16)
        assert waves[-1][1]["s1"] == n
        assert all(a[1]["s1"] == b[1]["s0"] for a, b in zip(waves, waves[1:]))
        parts = {w["part"] for _, w in waves}
        if row in rows:
            assert waves[0][1]["s0"] == shared_blocks  # the tail only
            if parts == {FOLD}:
                assert len({g for g, _ in waves}) == 1, "a folding segment cut across work-groups"
                assert {w["nparts"] for _, w in waves} == {ks}
                (pidx,) = {w["pidx"] for _, w in waves}
                pidx_of[(row, h)] = pidx
            else:
                cut += 1
                np_ = len(parts)
                assert parts == set(range(np_)) and np_ > 1
                nm, base, xb, xn = units.pop((int(qs[row]), h))
                assert nm == np_ and xn == ks
                assert {w["pidx"] for _, w in waves} == set(range(base, base + np_))
                pidx_of[(row, h)] = xb
        else:
            assert waves[0][1]["s0"] == 0
            assert FOLD not in parts
    return pidx_of, cut


def test_schedule_shared_prefix_units(lib):
    """Decode rows whose block tables start with the same blocks: the common
    prefix is attended by prefix units (the first units of the prefill
    section) once per query block, cut into key splits that tile it; each
    row's decode segment starts after the prefix and folds the partials the
    splits write for its query (itself, or through its merge unit when the
    planner cut it), which no other unit uses.  Rows below the group size,
    or a prefill row between decode rows, get no prefix."""
    import numpy as np

    hq, hkv, d, G = 32, 8, 128, 4
    pq = 4 * 16 * 2 // G  # queries per prefix unit at D=128 (4 waves x 32 m-rows / G): 32
    nqb = -(-70 // pq)
    q_lens = [40] + [1] * 70 + [1] * 2 + [1] * 3
    k_lens = [100] + [1500 + 37 * i for i in range(70)] + [900, 2100] + [800, 810, 820]
    offs = [60] + [k - 1 for k in k_lens[1:]]
    rows = len(q_lens)
    mb = max(-(-k // 16) for k in k_lens)
    bt = np.arange(rows * mb, dtype=np.int32).reshape(rows, mb) + 1000
    bt[1:71, :70] = 500000 + np.arange(70)  # 70 shared blocks: 1120 keys
    bt[73:76, :40] = 600000 + np.arange(40)  # only three rows: no group
    dec, pre, merge, ws, qs, npx = _schedule(lib, q_lens, k_lens, offs, hq=hq, hkv=hkv, d=d, bt=bt, prefix=True)
    assert npx > 0 and npx % (nqb * hkv) == 0  # every query block of the 70 rows, every kv head
    ks = npx // (nqb * hkv)
    assert 1 <= ks <= 1120 // 128
    pb = G * (d + 1) * 4
    nparts_total = ws // pb
    assert ws == nparts_total * pb
    pidx_of, _ = _shared_prefix_segments(dec, merge, qs, set(range(1, 71)), k_lens, hkv, 70, ks)
    assert len(pidx_of) == 70 * hkv
    # prefix units: (row, kv head, k0, k1), (query token, queries, partial, stride)
    pfx = pre[:npx].reshape(-1, 2, 4)
    rest = pre[npx:].reshape(-1, 2, 4)  # the prefill row's units follow: its 40 queries in two blocks
    assert len(rest) == 2 * hkv and all(u[0][0] == 0 and not u[1].any() for u in rest)
    tiles = {}
    written = []
    for (r0, h, k0, k1), (qtok, nq, base, stride) in pfx.tolist():
        assert r0 == 1 and 0 <= k0 < k1 <= 1120 and k0 % 32 == 0 and k1 % 32 == 0
        first = qtok - int(qs[1])
        assert first % pq == 0 and nq == min(pq, 70 - first)
        tiles.setdefault((first, h), []).append((k0, k1, base))
        for i in range(nq):
            written.append((first + 1 + i, h, base + i * stride))
    for (first, h), ranges in tiles.items():
        ranges.sort()
        assert ranges[0][0] == 0 and ranges[-1][1] == 1120 and len(ranges) == ks
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
    # split k of (row, h) writes partial pidx + k: exactly the ones the row's decode folds
    by_row = {}
    for row, h, p in written:
        by_row.setdefault((row, h), []).append(p)
    assert set(by_row) == set(pidx_of)
    for key, ps in by_row.items():
        assert sorted(ps) == list(range(pidx_of[key], pidx_of[key] + ks))
    fold_parts = [p for ps in by_row.values() for p in ps]
    merge_parts = [b + j for _, _, n, b, *_ in merge.tolist() for j in range(n)]
    allp = fold_parts + merge_parts
    assert len(set(allp)) == len(allp) and max(allp) < nparts_total


def test_schedule_fixed_partitions_give_work_groups_several_ranges_per_wave(lib):
    """A launch list of fixed partitions (16 rows x 32768 keys, 512-token
    partitions, as the long-context workload) gives each decode work-group up
    to four ranges per wave, one partition each, so that a device-full of
    work-groups takes the call in one round: 256 work-groups of 32 ranges,
    1024 slices each.  Without fixed partitions the same rows keep one range
    per wave."""
    rows, keys, pt = 16, 32768, 512
    k_lens = [keys] * rows
    dec, pre, merge, ws, qs = _schedule(lib, [1] * rows, k_lens, [k - 1 for k in k_lens], pt=pt)
    P = 4 * W
    assert len(dec) == GROUPS * P and all(w is not None for w in dec)
    _check_decode_schedule(dec, merge, ws, qs, W, {r: keys for r in range(rows)}, 8, pt=pt)
    for g in range(0, len(dec), P):
        ranges = dec[g:g + P]
        assert sum(w["s1"] - w["s0"] for w in ranges) == keys * rows * 8 // 16 // GROUPS
        # one partition per range
        assert all(w["s1"] - w["s0"] == pt // 16 and w["s0"] == w["part"] * pt // 16 for w in ranges)
    assert sorted(merge[:, 2].tolist()) == [keys // pt] * (rows * 8)
    # a few short rows: their work-groups are padded to 32 ranges with empty ones
    dec, pre, merge, ws, qs = _schedule(lib, [1, 1, 1], [300, 40, 2000], [299, 39, 1999], pt=64)
    assert len(dec) % P == 0
    _check_decode_schedule(dec, merge, ws, qs, W, {0: 300, 1: 40, 2: 2000}, 8, pt=64)
    # the planner's own split: one range per wave
    dec, pre, merge, ws, qs = _schedule(lib, [1] * rows, k_lens, [k - 1 for k in k_lens])
    assert len(dec) == GROUPS * W


def test_schedule_long_rows_sharing_a_short_prefix_fill_the_device(lib):
    """A few long rows whose tables share a short prefix: their tails are cut
    across work-groups like unshared rows (the prefix partials join each cut
    tail's merge unit), so the decode launch still fills a device's worth of
    work-groups with even loads."""
    import numpy as np

    for nrows, shared in ((4, 32), (8, 16), (16, 24)):
        k_lens = [16384] * nrows
        mb = 16384 // 16
        bt = np.arange(nrows * mb, dtype=np.int32).reshape(nrows, mb) + 1000
        bt[:, :shared] = 7 + np.arange(shared)
        dec, pre, merge, ws, qs, npx = _schedule(lib, [1] * nrows, k_lens, [k - 1 for k in k_lens], bt=bt,
                                                 prefix=True)
        assert npx > 0
        ks = npx // 8  # one query block, 8 kv heads
        ngroups = len(dec) // W
        loads = [sum(w["s1"] - w["s0"] for w in dec[g:g + W] if w is not None) for g in range(0, len(dec), W)]
        total = nrows * 8 * (mb - shared)
        assert sum(loads) == total
        assert ngroups >= GROUPS - 8, (nrows, ngroups)
        assert max(loads) <= total / GROUPS + 16, (nrows, max(loads), total / GROUPS)
        pidx_of, cut = _shared_prefix_segments(dec, merge, qs, set(range(nrows)), k_lens, 8, shared, ks)
        assert cut > 0 and len(pidx_of) == nrows * 8
        # every prefix partial a row needs is written by a prefix unit (query
        # token = row here: one query per row from token 0)
        written = set()
        for (r0, h, k0, k1), (qtok, nq, base, stride) in pre[:npx].reshape(-1, 2, 4).tolist():
            for i in range(nq):
                written.add((qtok + i, h, base + i * stride))
        for (row, h), p in pidx_of.items():
            assert all((row, h, p + k) in written for k in range(ks))


def test_schedule_prefix_group_keeps_the_longer_prefix(lib):
    """8 rows sharing 4096 keys, then a row that shares only their first 256:
    the ninth row does not join (it would cut every row's shared keys to
    256), so the group keeps its 4096-key prefix."""
    import numpy as np

    k_lens = [5000] * 9
    mb = -(-5000 // 16)
    bt = np.arange(9 * mb, dtype=np.int32).reshape(9, mb) + 1000
    bt[:8, :256] = 7 + np.arange(256)
    bt[8, :16] = 7 + np.arange(16)
    dec, pre, merge, ws, qs, npx = _schedule(lib, [1] * 9, k_lens, [k - 1 for k in k_lens], bt=bt, prefix=True)
    ranges = {(k0, k1) for (r0, h, k0, k1) in pre[:npx].reshape(-1, 2, 4)[:, 0].tolist()}
    assert min(k0 for k0, _ in ranges) == 0 and max(k1 for _, k1 in ranges) == 4096
    assert 8 not in {w["row"] for w in dec if w is not None and w["part"] == FOLD}
    # the ninth row reads all its keys itself
    starts = [w["s0"] for w in dec if w is not None and w["row"] == 8]
    assert min(starts) == 0


def test_schedule_shared_prefix_needs_enough_keys(lib):
    """Shared blocks covering fewer than 256 keys before a row's last key,
    or a fixed partition size, leave the rows without prefix units."""
    import numpy as np

    k_lens = [1000] * 8
    bt = np.arange(8 * 63, dtype=np.int32).reshape(8, 63) + 1000
    bt[:, :15] = 7  # 240 shared keys
    *_, npx = _schedule(lib, [1] * 8, k_lens, [k - 1 for k in k_lens], bt=bt, prefix=True)
    assert npx == 0
    bt[:, :16] = 7  # 256
    *_, npx = _schedule(lib, [1] * 8, k_lens, [k - 1 for k in k_lens], bt=bt, prefix=True)
    assert npx > 0
    *_, npx = _schedule(lib, [1] * 8, k_lens, [k - 1 for k in k_lens], bt=bt, prefix=True, pt=256)
    assert npx == 0
    # the prefix must end before every row's last key: a 257-key row caps it at 256
    k_lens = [1000] * 7 + [257]
    bt[:, :62] = 7
    *_, npx = _schedule(lib, [1] * 8, k_lens, [k - 1 for k in k_lens], bt=bt, prefix=True)
    assert npx > 0


def test_schedule_shared_prefix_stays_within_one_device_fill(lib):
    """256 rows sharing 64 blocks with private tails of 64..512 keys (the
    prefix-sharing workload's shape): the tails, which are never cut, are
    packed into at most one device-full of decode work-groups (256 of 8
    waves where no device is visible) with balanced loads."""
    import numpy as np

    rng = np.random.default_rng(4)
    tails = rng.integers(64, 512, size=256, endpoint=True)
    k_lens = [1024 + int(t) for t in tails]
    mb = max(-(-k // 16) for k in k_lens)
    bt = np.arange(256 * mb, dtype=np.int32).reshape(256, mb) + 1000
    bt[:, :64] = 7 + np.arange(64)
    dec, pre, merge, ws, qs, npx = _schedule(lib, [1] * 256, k_lens, [k - 1 for k in k_lens], bt=bt, prefix=True)
    assert npx > 0 and len(merge) == 0
    assert len(dec) <= W * GROUPS and len(dec) % W == 0
    loads = [sum(w["s1"] - w["s0"] for w in dec[g:g + W] if w is not None) for g in range(0, len(dec), W)]
    total = sum(-(-k // 16) - 64 for k in k_lens) * 8
    assert sum(loads) == total
    assert max(loads) <= total / len(loads) + 32  # within one tail of the mean


def test_schedule_attn_flags(lib):
    """The schedule takes the attention call's attn_flags: the deterministic
    bit leaves the plan as it is, unknown bits are rejected."""
    import numpy as np

    k_lens = [300, 1200, 17]
    plans = [_schedule(lib, [1, 1, 1], k_lens, [k - 1 for k in k_lens], causal=c) for c in (1, 3)]
    assert all(np.array_equal(a, b) for a, b in zip(plans[0][1:3], plans[1][1:3]))
    assert plans[0][0] == plans[1][0] and plans[0][3] == plans[1][3]
    q = np.ones(1, np.int32)
    cnt = [ctypes.c_int64() for _ in range(5)]
    got = lib.kvhot_paged_attention_schedule(q.ctypes.data, q.ctypes.data, q.ctypes.data, q.ctypes.data,
                                             q.ctypes.data, 1, 1, 32, 8, 128, 16, 0, 8, 2, None, 0,
                                             *(ctypes.byref(c) for c in cnt))
    assert got == -1 and b"attn_flags" in lib.kvhot_last_error()
