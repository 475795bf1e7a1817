"""Per-step admission: which requests run this step, how many prompt tokens
each prefill row computes, and who is evicted when the pool runs dry
(serving_engine/scheduler.py:25-187).

Same policy as the reference's Scheduler:
* running requests are considered before waiting ones;
* a decode row costs one token and needs room for it (can_append_slot); a
  prefill row is gated on min(min_chunk_size, remaining) tokens of budget and
  then takes as much of the remaining budget as it has tokens left;
* the token cap only stops adding work on top of work already batched, so a
  lone candidate larger than the cap still runs;
* a fresh (or preempted) prefill needs blocks for all its tokens; a running
  one already holds them;
* only when nothing at all was scheduled and a decode row is blocked on the
  pool is the most recently admitted other running request preempted (LIFO)
  to let that row through.
On top of it, the step's copy-on-write pairs go out in
SchedulerOutput.blocks_to_copy (block_manager.BlockManager.prepare_write).
"""
from __future__ import annotations

from typing import List, Optional

from .block_manager import BlockManager
from .request import Request, RequestPhase, RequestStatus, SchedulerOutput


class Scheduler:
    def __init__(self, block_manager: BlockManager, max_num_batched_tokens: Optional[int] = None,
                 max_num_seqs: Optional[int] = None, min_chunk_size: Optional[int] = None):
        self.block_manager = block_manager
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_seqs = max_num_seqs
        self.min_chunk_size = min_chunk_size
        self.waiting: List[Request] = []
        self.running: List[Request] = []

    def add_request(self, request: Request) -> None:
        self.block_manager.match_prefix(request)
        self.waiting.append(request)

    def _victim(self, keep: Request) -> Optional[Request]:
        """The most recently admitted running request other than `keep`."""
        return next((r for r in reversed(self.running) if r is not keep), None)

    def _over_budget(self, used: int, cost: int) -> bool:
        cap = self.max_num_batched_tokens
        return cap is not None and used > 0 and used + cost > cap

    def schedule(self) -> SchedulerOutput:
        out = SchedulerOutput()
        bm = self.block_manager
        blocked: List[Request] = []
        used = 0  # tokens batched this step
        for req in self.running + self.waiting:
            if self.max_num_seqs is not None and len(out.scheduled_requests) >= self.max_num_seqs:
                break
            left = req.total_len - req.num_computed_tokens
            decode = req.phase == RequestPhase.NEEDS_DECODE
            if decode:
                gate = 1
            else:
                gate = left if self.min_chunk_size is None else min(self.min_chunk_size, left)
            if self._over_budget(used, gate):
                continue
            if decode:
                if not bm.can_append_slot(req):
                    blocked.append(req)
                    continue
                bm.append_slot(req)
                out.scheduled_requests.append(req)
                used += 1
                continue
            admitted = req.status == RequestStatus.RUNNING
            if not admitted and not bm.can_allocate(req):
                continue
            chunk = left if self.max_num_batched_tokens is None else min(left, self.max_num_batched_tokens - used)
            start = req.num_computed_tokens
            if admitted:
                # shared blocks this chunk writes are copied first
                if bm.shared_blocks_in(req, start, start + chunk) > bm.get_num_free_blocks():
                    continue
            else:
                bm.allocate(req)
                req.status = RequestStatus.RUNNING
                self.waiting = [r for r in self.waiting if r is not req]
                self.running.append(req)
            bm.prepare_write(req, start, start + chunk)
            out.scheduled_requests.append(req)
            out.prefill_chunk_sizes[req.request_id] = chunk
            if start + chunk >= req.total_len:
                out.prefill_final_chunk.add(req.request_id)
            used += chunk

        if not out.scheduled_requests and blocked:
            # The pool is exhausted and nothing advanced: evict one request so
            # the first blocked decode row can take its next token.
            row = blocked[0]
            victim = self._victim(row)
            if victim is not None:
                bm.preempt(victim)
                self.running.remove(victim)
                self.waiting.append(victim)
                out.preempted_requests.append(victim)
                if bm.can_append_slot(row):
                    bm.append_slot(row)
                    out.scheduled_requests.append(row)
        out.blocks_to_copy = bm.take_copies()
        return out

    def update_after_step(self, scheduler_output: SchedulerOutput) -> None:
        """After the step's tokens were appended to output_token_ids: a
        request that reached max_new_tokens or sampled EOS finishes and frees
        its blocks; a prefill row advances by its chunk, registers its newly
        computed prompt blocks, and turns to decode after its final chunk."""
        bm = self.block_manager
        for req in scheduler_output.scheduled_requests:
            out_ids = req.output_token_ids
            if out_ids and (len(out_ids) >= req.max_new_tokens or out_ids[-1] == req.eos_token_id):
                req.status = RequestStatus.FINISHED
                bm.free(req)
                self.running = [r for r in self.running if r is not req]
            elif req.phase == RequestPhase.NEEDS_PREFILL:
                req.num_computed_tokens += scheduler_output.prefill_chunk_sizes[req.request_id]
                bm.register_computed_blocks(req)
                if req.request_id in scheduler_output.prefill_final_chunk:
                    req.phase = RequestPhase.NEEDS_DECODE

    def has_unfinished_requests(self) -> bool:
        return bool(self.waiting or self.running)
