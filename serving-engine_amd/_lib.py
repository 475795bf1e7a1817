"""ctypes binding of libkvhot.so, the C-ABI library declared in include/kvhot.h.

torch is imported before the library is opened so that libkvhot binds to the
HIP runtime torch already loaded (both carry SONAME libamdhip64.so.7): device
pointers and hipStream_t handles from torch are then valid inside the library.

There is no fallback: if the library is missing or fails to load, every call
raises.  Build it with `python serving-engine_amd/build.py` (or
`__graft_entry__.build()`).
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before libkvhot, see above)

# KVHOT_LIB may name another build of the same library (e.g. a tuning variant).
LIB_PATH = os.environ.get("KVHOT_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                       "libkvhot.so")

KVHOT_F32 = 0
KVHOT_F16 = 1
KVHOT_BF16 = 2

# attn_flags bits
KVHOT_CAUSAL = 1
KVHOT_DETERMINISTIC = 2
KVHOT_VERIFY_BLOCKS = 4

# Split-K partials kvhot_paged_attention_noalloc holds (KVHOT_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 64 << 20

_DTYPE_CODES = {
    torch.float32: KVHOT_F32,
    torch.float16: KVHOT_F16,
    torch.bfloat16: KVHOT_BF16,
}

# Every symbol include/kvhot.h declares, with its ctypes signature.
_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)

SIGNATURES = {
    "kvhot_version": (_int, []),
    "kvhot_last_error": (ctypes.c_char_p, []),
    "kvhot_reshape_and_cache": (
        _int,
        [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _int,
         _i64, _i64, _i64, _i64, _i64, _int, _vp],
    ),
    "kvhot_copy_blocks": (
        _int,
        [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp],
    ),
    "kvhot_build_slot_mapping": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp],
    ),
    "kvhot_paged_attention_workspace_bytes": (
        _i64,
        [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int],
    ),
    "kvhot_paged_attention_schedule": (
        _i64,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _vp, _i64,
         _i64p, _i64p, _i64p, _i64p, _i64p],
    ),
    "kvhot_paged_attention": (
        _int,
        [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
         _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, ctypes.c_float, _int, _int, _i64, _vp, _i64, _i64, _i64, _i64,
         _i64, _vp, _i64, _vp],
    ),
    "kvhot_paged_attention_noalloc": (
        _int,
        [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
         _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, ctypes.c_float, _int, _int, _i64, _vp, _i64, _i64, _i64, _i64,
         _i64, _vp],
    ),
}


class KvhotError(RuntimeError):
    """A libkvhot entry point returned a nonzero status."""


_LIB = None


def load() -> ctypes.CDLL:
    """Opens libkvhot.so once and binds every declared symbol; raises if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python serving-engine_amd/build.py`"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def i64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().kvhot_last_error().decode(errors="replace")
        raise KvhotError(f"{what} failed with status {status}: {msg}")


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (as an integer)."""
    return torch.cuda.current_stream(device).cuda_stream
