"""Requests and the per-step batch, as the reference engine defines them
(serving_engine/request.py:9-64, serving_engine/scheduler.py:8-22).

The hot path only reads a request's lengths, phase and block table, and is
duck-typed on them: any object with the same attribute names works, including
the reference's own Request and SchedulerOutput (whose phase enum is matched
by member name).  The rest of the fields serve the block manager and the
scheduler (block_manager.py, scheduler.py).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Dict, List, Optional, Set, Tuple


class RequestPhase(Enum):
    NEEDS_PREFILL = auto()
    NEEDS_DECODE = auto()


class RequestStatus(Enum):
    WAITING = auto()    # not admitted yet (or back from a preemption)
    RUNNING = auto()    # admitted: holds blocks
    PREEMPTED = auto()  # evicted; its blocks were freed and it recomputes
    FINISHED = auto()


@dataclass
class Request:
    request_id: str
    prompt_token_ids: List[int]
    max_new_tokens: int = 256
    eos_token_id: Optional[int] = None
    output_token_ids: List[int] = field(default_factory=list)
    phase: RequestPhase = RequestPhase.NEEDS_PREFILL
    status: RequestStatus = RequestStatus.WAITING
    # logical block index -> physical block id
    block_table: List[int] = field(default_factory=list)
    # tokens of this request whose K/V are already in the cache
    num_computed_tokens: int = 0
    arrival_time: float = field(default_factory=time.monotonic)

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def output_len(self) -> int:
        return len(self.output_token_ids)

    @property
    def total_len(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    @property
    def is_finished(self) -> bool:
        return self.status == RequestStatus.FINISHED

    def all_token_ids(self) -> List[int]:
        return self.prompt_token_ids + self.output_token_ids


@dataclass
class SchedulerOutput:
    scheduled_requests: List[Request] = field(default_factory=list)
    preempted_requests: List[Request] = field(default_factory=list)
    # request_id -> tokens prefilled this step (prefill rows only)
    prefill_chunk_sizes: Dict[str, int] = field(default_factory=dict)
    # prefill rows whose chunk completes their prompt, decided at schedule time
    prefill_final_chunk: Set[str] = field(default_factory=set)
    # (src, dst) block copies to run before this step's K/V appends:
    # copy-on-write of shared blocks a scheduled row writes into
    blocks_to_copy: List[Tuple[int, int]] = field(default_factory=list)


def is_prefill(req) -> bool:
    """True for a NEEDS_PREFILL request, for this module's enum or any enum
    with the same member names (serving_engine/request.py:9-16)."""
    return getattr(req.phase, "name", None) == "NEEDS_PREFILL"
