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
    assert len(names) == 7
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
            4, 4, 1, 100, 32, 8, 128, 16, 64, 0.1, 1, 2, 0, None, 0, None]
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
