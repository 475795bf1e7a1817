"""The request/batch fields the KV-cache hot path reads.

Mirrors the reference's data types only as far as the hot path consumes them
(serving_engine/request.py:9-64, serving_engine/scheduler.py:8-22).  The hot
path is duck-typed on them: any object with the same attribute names works,
including the reference's own Request and SchedulerOutput, whose phase enum is
matched by member name.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Dict, List, Set


class RequestPhase(Enum):
    NEEDS_PREFILL = auto()
    NEEDS_DECODE = auto()


@dataclass
class Request:
    request_id: str
    prompt_token_ids: List[int]
    output_token_ids: List[int] = field(default_factory=list)
    phase: RequestPhase = RequestPhase.NEEDS_PREFILL
    # logical block index -> physical block id
    block_table: List[int] = field(default_factory=list)
    # tokens of this request whose K/V are already in the cache
    num_computed_tokens: int = 0

    @property
    def prompt_len(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def total_len(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    def all_token_ids(self) -> List[int]:
        return self.prompt_token_ids + self.output_token_ids


@dataclass
class SchedulerOutput:
    scheduled_requests: List[Request] = field(default_factory=list)
    # request_id -> tokens prefilled this step (prefill rows only)
    prefill_chunk_sizes: Dict[str, int] = field(default_factory=dict)
    prefill_final_chunk: Set[str] = field(default_factory=set)


def is_prefill(req) -> bool:
    """True for a NEEDS_PREFILL request, for this module's enum or any enum
    with the same member names (serving_engine/request.py:9-16)."""
    return getattr(req.phase, "name", None) == "NEEDS_PREFILL"
