"""Paged KV-cache geometry shared with the reference engine.

BLOCK_SIZE = 16 tokens per physical block (serving_engine/block.py:7).  Block
ids index dim 2 of the whole-pool tensor kv_cache[L, 2, N, BLOCK_SIZE, Hkv, D]
(serving_engine/model_runner.py:101-110).
"""

BLOCK_SIZE = 16

BlockId = int


class Block:
    """One physical block of the pool: how many block tables hold it, and,
    once its prompt tokens are computed and registered for prefix matching,
    the chained key it is found under (serving_engine/block.py:12-24)."""

    __slots__ = ("block_id", "ref_count", "content_hash")

    def __init__(self, block_id: BlockId, ref_count: int = 1, content_hash=None):
        self.block_id = block_id
        self.ref_count = ref_count
        self.content_hash = content_hash

    def __repr__(self):
        return f"Block({self.block_id}, ref_count={self.ref_count}, content_hash={self.content_hash})"
