"""Paged KV-cache geometry shared with the reference engine.

BLOCK_SIZE = 16 tokens per physical block (serving_engine/block.py:7).  Block
ids index dim 2 of the whole-pool tensor kv_cache[L, 2, N, BLOCK_SIZE, Hkv, D]
(serving_engine/model_runner.py:101-110).
"""

BLOCK_SIZE = 16

BlockId = int
