"""MI355X-native KV-cache hot path of a paged-attention serving engine.

Drop-in for the hot path of the reference engine (ayush-os/serving-engine):
paged attention, KV append, block copy and step metadata run as hand-written
gfx950 HIP kernels in libkvhot.so (C ABI: include/kvhot.h), called through
ctypes.  BlockManager and Scheduler restate the reference's block pool and
admission policy on the host, with copy-on-write of shared blocks.  The directory name is not a Python identifier, so import it with
``importlib.import_module("serving-engine_amd")``.
"""
from .block import BLOCK_SIZE
from .paged_attention_kernel import (
    PAGED_K_TILE_SIZE,
    PAGED_Q_TILE_SIZE,
    build_paged_batch_metadata,
    build_slot_mapping,
    paged_flash_attention,
)
from .model_runner import (
    PAGED_HIP_ATTN_IMPL,
    POOL_LAYOUTS,
    _PagedKVCache,
    allocate_kv_cache,
    forward_step,
    hip_paged_attention_forward,
    num_blocks_for_memory,
    register_attention,
    sample_step,
    step_inputs,
    step_token_ids,
)
from .decode_graph import DecodeStepGraph
from .request import Request, RequestPhase, RequestStatus, SchedulerOutput
from .block_manager import BlockManager
from .scheduler import Scheduler

__all__ = [
    "BLOCK_SIZE",
    "BlockManager",
    "DecodeStepGraph",
    "PAGED_K_TILE_SIZE",
    "PAGED_Q_TILE_SIZE",
    "PAGED_HIP_ATTN_IMPL",
    "Request",
    "RequestPhase",
    "RequestStatus",
    "Scheduler",
    "SchedulerOutput",
    "_PagedKVCache",
    "POOL_LAYOUTS",
    "allocate_kv_cache",
    "build_paged_batch_metadata",
    "build_slot_mapping",
    "forward_step",
    "hip_paged_attention_forward",
    "num_blocks_for_memory",
    "paged_flash_attention",
    "register_attention",
    "sample_step",
    "step_inputs",
    "step_token_ids",
]
