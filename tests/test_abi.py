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
            4, 4, 1, 100, 32, 8, 128, 16, 64, 0.1, 1, 2, 64, None, 0, 0, None, 0, None]
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


def test_workspace_bytes(lib):
    # decode: 64 rows, max ctx 2048, 32/8 heads, D=128, 256-token partitions
    # -> LSE 64*32*8*4 B, partials 64*32*8*128*4 B
    n = lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 32, 8, 128, 16, 256, 2)
    assert n == 65536 + 64 * 32 * 8 * 128 * 4
    # one partition: no workspace
    assert lib.kvhot_paged_attention_workspace_bytes(4, 4, 1, 130, 12, 12, 64, 16, 512, 2) == 0
    # fp32 runs the VALU kernel, which never splits
    assert lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 32, 8, 128, 16, 256, 0) == 0
    assert lib.kvhot_paged_attention_workspace_bytes(64, 64, 1, 2048, 30, 8, 128, 16, 256, 2) < 0


def _schedule(lib, q_lens, k_lens, offs, hq=32, hkv=8, d=128, pt=0, causal=1, dtype=2):
    import numpy as np

    q = np.asarray(q_lens, np.int32)
    k = np.asarray(k_lens, np.int32)
    o = np.asarray(offs, np.int32)
    qs = np.concatenate([[0], np.cumsum(q)[:-1]]).astype(np.int32)
    mb = max(-(-int(x) // 16) for x in k)
    bt = (np.arange(len(q) * mb, dtype=np.int32).reshape(len(q), mb) + 1000)  # block ids 1000 + r*mb + j
    nd, npf, ptu = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    outs = (ctypes.byref(nd), ctypes.byref(npf), ctypes.byref(ptu))
    head = (q.ctypes.data, k.ctypes.data, qs.ctypes.data, o.ctypes.data, bt.ctypes.data, mb, len(q), hq, hkv,
            d, 16, pt, causal, dtype)
    total = lib.kvhot_paged_attention_schedule(*head, None, 0, *outs)
    units = np.zeros((max(total, 0), 8), np.int32)
    got = lib.kvhot_paged_attention_schedule(*head, units.ctypes.data, total, *outs)
    assert got == total
    # decode descriptors carry (query token, visible keys, first block, query position)
    for row, kvh, s0, s1, qtok, kend, first, qpos in units[:nd.value].tolist():
        if row >= 0:
            assert qtok == qs[row] and qpos == o[row] and kend == min(k[row], o[row] + 1)
            assert first == 1000 + row * mb + (16 * s0) // 16
    return units[:, :4], nd.value, npf.value, ptu.value


def _check_decode_schedule(dec, waves_per_group, rows, hkv, pt, max_slices):
    """Every (row, kv head, partition) of every decode row is covered exactly
    once by contiguous waves of one work-group; no wave walks more than
    max_slices slices."""
    assert len(dec) % waves_per_group == 0
    cover = {}
    for g0 in range(0, len(dec), waves_per_group):
        grp = dec[g0:g0 + waves_per_group]
        seen_keys = set()
        prev = None
        for row, kvh, s0, s1 in grp.tolist():
            if row < 0:
                prev = None
                continue
            assert s1 - s0 <= max_slices
            key = (row, kvh, (16 * s0) // pt)
            if key != prev:
                assert key not in seen_keys, "segment split inside a work-group"
                seen_keys.add(key)
            prev = key
            cover.setdefault(key, []).append((s0, s1))
    for row, kend in rows.items():
        nparts = max(-(-kend // pt), 1)
        for p in range(nparts):
            kb, ke = p * pt, min(kend, (p + 1) * pt)
            for h in range(hkv):
                pieces = sorted(cover.pop((row, h, p)))
                assert pieces[0][0] == kb // 16 and pieces[-1][1] == kb // 16 + -(-(ke - kb) // 16)
                assert all(a[1] == b[0] for a, b in zip(pieces, pieces[1:]))
    assert not cover


def test_schedule_lists_every_unit_once(lib):
    """Host planner: decode waves cover every (row, kv head, partition) once,
    balanced; prefill units every (row, kv head, query block); longest first."""
    # rows: decode 300 keys, decode 40 keys, prefill 20 queries on 50 keys, empty chunk, decode 2000 keys
    q_lens, k_lens, offs = [1, 1, 20, 0, 1], [300, 40, 50, 16, 2000], [299, 39, 30, 16, 1999]
    units, nd, npf, ptu = _schedule(lib, q_lens, k_lens, offs, pt=1024)
    assert ptu == 1024
    dec, pre = units[:nd], units[nd:]
    assert len(pre) == npf
    # 1024-key partitions over 16-wave groups: at most 1024 / 16 / 16 = 4 slices per wave
    _check_decode_schedule(dec, 16, {0: 300, 1: 40, 4: 2000}, 8, 1024, 4)
    # prefill: 20 queries, 16 per block (64 m-rows / G=4) -> 2 blocks x 8 kv heads; the empty chunk has none
    assert sorted(map(tuple, pre[:, :3].tolist())) == sorted((2, h, b) for h in range(8) for b in range(2))
    # the second block (queries 16..19 at positions 46..49) sees 50 keys, the first 46
    assert sorted(set(pre[:, 3].tolist())) == [3, 4]
    assert list(pre[:, 3]) == sorted(pre[:, 3], reverse=True)


def test_schedule_chooses_partition_for_whole_batch(lib):
    """Without a partition size the planner keeps every row in one partition
    when the batch fits, with at least 8 slices per wave."""
    import numpy as np

    rng = np.random.default_rng(0)
    ctx = rng.integers(128, 2048, size=64, endpoint=True)
    units, nd, npf, ptu = _schedule(lib, [1] * 64, ctx, ctx - 1)
    assert npf == 0 and ptu >= 2048 and ptu % 256 == 0
    _check_decode_schedule(units[:nd], 16, dict(enumerate(ctx.tolist())), 8, ptu, ptu // 256)


def test_schedule_empty_for_vector_path(lib):
    # fp32 runs the VALU kernel: no launch list
    units, nd, npf, _ = _schedule(lib, [1, 1], [100, 50], [99, 49], dtype=0)
    assert len(units) == 0 and nd == 0 and npf == 0
