"""Block pool bookkeeping for the paged KV cache: free list, block tables,
reference counts, chained-hash prefix matching, preemption
(serving_engine/block_manager.py:7-141), plus copy-on-write.

Same interface and observable behaviour as the reference's BlockManager:
block ids are handed out from the top of the pool down (the free list is a
stack over range(N)), a block is matched for a prefix only as part of an
unbroken chain of full prompt blocks from the start, the first block
registered under a key stays its canonical holder, and a block returns to
the pool (and leaves the prefix index) when its last holder frees it.

Copy-on-write (no counterpart in the reference, which shares a forked
request's partly filled last block and lets both requests append into it):
before a step writes a token into a block that another block table also
holds, the writer gets a private copy.  The block manager swaps the new id
into the writer's table and queues (src, dst); the scheduler hands the queue
to the step (SchedulerOutput.blocks_to_copy), which copies the blocks on the
GPU (_PagedKVCache.copy_blocks, one launch for every layer, K and V) before
the step's K/V appends.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

from .block import BLOCK_SIZE, Block
from .request import Request, RequestPhase, RequestStatus


def chain_key(parent: Optional[int], tokens) -> int:
    """Prefix-index key of a full block of prompt tokens: its tokens together
    with the key of the block before it, since a block's K/V depend on every
    earlier token, not only on its own."""
    return hash((parent, tuple(tokens)))


class BlockManager:
    def __init__(self, num_gpu_blocks: int, block_size: int = BLOCK_SIZE):
        if num_gpu_blocks < 0 or block_size <= 0:
            raise ValueError("num_gpu_blocks must be >= 0 and block_size > 0")
        self.num_gpu_blocks = num_gpu_blocks
        self.block_size = block_size
        self.blocks = [Block(i, 0) for i in range(num_gpu_blocks)]
        self.free_blocks: List[int] = list(range(num_gpu_blocks))  # a stack: pops the highest id
        self.hash_to_block: dict = {}
        self.pending_copies: List[Tuple[int, int]] = []

    # -- pool ---------------------------------------------------------------

    def get_num_free_blocks(self) -> int:
        return len(self.free_blocks)

    def _take(self) -> int:
        block_id = self.free_blocks.pop()
        self.blocks[block_id].ref_count += 1
        return block_id

    def _drop(self, block_id: int) -> None:
        block = self.blocks[block_id]
        block.ref_count -= 1
        if block.ref_count == 0:
            self.free_blocks.append(block_id)
            if block.content_hash is not None:
                # Only a canonical block carries a key (first holder wins),
                # so the index entry is this block's.
                del self.hash_to_block[block.content_hash]
                block.content_hash = None

    def _missing_blocks(self, request: Request) -> int:
        return -(-request.total_len // self.block_size) - len(request.block_table)

    # -- prefix cache -------------------------------------------------------

    def match_prefix(self, request: Request) -> None:
        """Takes the longest run of the prompt's full blocks, from the first,
        whose chained keys are in the index; the request starts with those
        tokens computed."""
        bs = self.block_size
        key = None
        for i in range(request.prompt_len // bs):
            key = chain_key(key, request.prompt_token_ids[i * bs:(i + 1) * bs])
            hit = self.hash_to_block.get(key)
            if hit is None:
                break
            request.block_table.append(hit)
            self.blocks[hit].ref_count += 1
        request.num_computed_tokens = len(request.block_table) * bs

    def register_computed_blocks(self, request: Request) -> None:
        """Enters the request's full prompt blocks whose tokens are computed
        into the index.  A block that already has a key (registered earlier,
        or matched) passes its key on as the next block's parent; under a key
        that another block already holds, the first holder stays."""
        bs = self.block_size
        upto = min(request.num_computed_tokens, request.prompt_len) // bs
        key = None
        for i in range(upto):
            block = self.blocks[request.block_table[i]]
            if block.content_hash is not None:
                key = block.content_hash
                continue
            key = chain_key(key, request.prompt_token_ids[i * bs:(i + 1) * bs])
            if key not in self.hash_to_block:
                self.hash_to_block[key] = block.block_id
                block.content_hash = key

    # -- admission and growth -----------------------------------------------

    def can_allocate(self, request: Request) -> bool:
        return self._missing_blocks(request) <= self.get_num_free_blocks()

    def allocate(self, request: Request) -> None:
        """Blocks for every token of the request (total_len, so the tokens a
        preempted request already generated are covered too)."""
        assert self.can_allocate(request)
        for _ in range(self._missing_blocks(request)):
            request.block_table.append(self._take())

    def _has_capacity_for(self, request: Request) -> bool:
        # Measured against the table itself: a length on a block boundary
        # (a recompute, or a prompt of whole blocks) needs one more block for
        # its next token whatever the history.
        return len(request.block_table) * self.block_size >= request.total_len

    def _shared(self, request: Request, index: int) -> bool:
        return 0 <= index < len(request.block_table) and \
            self.blocks[request.block_table[index]].ref_count > 1

    def _next_write_shared(self, request: Request) -> bool:
        # A decode step writes position total_len - 1, unless it is already
        # computed (then nothing is written and nothing needs a copy).
        pos = request.total_len - 1
        return pos >= request.num_computed_tokens and self._shared(request, pos // self.block_size)

    def can_append_slot(self, request: Request) -> bool:
        """Room for the request's next token: free capacity in a block only
        it holds, or one free block (a new last block, or a private copy of a
        shared one)."""
        if self._has_capacity_for(request) and not self._next_write_shared(request):
            return True
        return self.get_num_free_blocks() >= 1

    def append_slot(self, request: Request) -> Optional[int]:
        """Makes room for the request's next token (position total_len - 1).
        Returns the id of a block newly placed in its table (a new last block
        or a private copy), else None."""
        if not self._has_capacity_for(request):
            assert self.can_append_slot(request)
            block_id = self._take()
            request.block_table.append(block_id)
            return block_id
        if not self._next_write_shared(request):
            return None
        copies = self.prepare_write(request, request.total_len - 1, request.total_len)
        return copies[-1][1]

    def shared_blocks_in(self, request: Request, start: int, end: int) -> int:
        """Blocks of the request's table holding tokens [start, end) that
        another table holds too."""
        bs = self.block_size
        return sum(self._shared(request, i) for i in range(start // bs, -(-end // bs)))

    def prepare_write(self, request: Request, start: int, end: int) -> List[Tuple[int, int]]:
        """Copy-on-write for a step that writes tokens [start, end) of the
        request: each block of that range that another table also holds is
        replaced in this table by a free block, and (src, dst) is queued for
        the step to copy.  Returns the pairs queued by this call."""
        bs = self.block_size
        made = []
        for i in range(start // bs, -(-end // bs)):
            if self._shared(request, i):
                assert self.get_num_free_blocks() >= 1, "no free block for a copy-on-write"
                src = request.block_table[i]
                dst = self._take()
                request.block_table[i] = dst
                self.blocks[src].ref_count -= 1  # still held elsewhere: never reaches 0 here
                made.append((src, dst))
        self.pending_copies.extend(made)
        return made

    def take_copies(self) -> List[Tuple[int, int]]:
        """The queued (src, dst) copies, which the caller now owns."""
        copies, self.pending_copies = self.pending_copies, []
        return copies

    # -- release ------------------------------------------------------------

    def free(self, request: Request) -> None:
        for block_id in request.block_table:
            self._drop(block_id)
        request.block_table = []

    def fork(self, parent: Request, child: Request) -> None:
        """The child shares every block of the parent's table (a copy of the
        list); a later write into a shared block copies it first."""
        child.block_table = list(parent.block_table)
        for block_id in child.block_table:
            self.blocks[block_id].ref_count += 1

    def preempt(self, request: Request) -> None:
        """Frees the request's blocks; it recomputes from its first token."""
        self.free(request)
        request.num_computed_tokens = 0
        request.phase = RequestPhase.NEEDS_PREFILL
        request.status = RequestStatus.PREEMPTED
