"""Host side of a step: the input tokens ModelRunner.forward feeds the model
(serving_engine/model_runner.py:150-163), rows in scheduled order."""
from conftest import sea_module


def test_step_token_ids_takes_chunks_and_last_tokens():
    sea = sea_module()
    so = sea.SchedulerOutput()
    a = sea.Request("a", list(range(100, 130)), max_new_tokens=4)   # prefill, chunk 2 of 3
    a.num_computed_tokens = 8
    b = sea.Request("b", [7, 8, 9], max_new_tokens=4, output_token_ids=[11, 12])  # decode
    b.phase = sea.RequestPhase.NEEDS_DECODE
    b.num_computed_tokens = 4
    c = sea.Request("c", [1, 2, 3, 4, 5], max_new_tokens=4)        # whole prompt in one chunk
    so.scheduled_requests += [a, b, c]
    so.prefill_chunk_sizes.update({"a": 10, "c": 5})
    assert sea.step_token_ids(so) == list(range(108, 118)) + [12] + [1, 2, 3, 4, 5]


def _step(sea, tables_and_lens):
    so = sea.SchedulerOutput()
    for i, (table, n) in enumerate(tables_and_lens):
        r = sea.Request(f"r{i}", list(range(n - 1)), max_new_tokens=4, output_token_ids=[0])
        r.phase = sea.RequestPhase.NEEDS_DECODE
        r.num_computed_tokens = n - 1
        r.block_table = list(table)
        so.scheduled_requests.append(r)
    return so


def test_metadata_checks_block_tables_against_the_pool():
    """With the pool size, a step's host block tables are checked before any
    copy: blocks outside the pool and tables too short for the keys read
    raise IndexError (the reference's index_copy_ raises on an out-of-pool
    write slot); without it nothing is checked."""
    import pytest

    sea = sea_module()
    ok = _step(sea, [([3, 7], 20), ([0], 16)])
    meta = sea.build_paged_batch_metadata(ok, device="cpu", num_blocks=8)
    assert meta["host_block_table"].tolist() == [[3, 7], [0, 0]]
    with pytest.raises(IndexError, match="outside the pool"):
        sea.build_paged_batch_metadata(_step(sea, [([3, 8], 20)]), device="cpu", num_blocks=8)
    with pytest.raises(IndexError, match="outside the pool"):
        sea.build_paged_batch_metadata(_step(sea, [([-1], 5)]), device="cpu", num_blocks=8)
    with pytest.raises(IndexError, match="covers 16 tokens"):
        sea.build_paged_batch_metadata(_step(sea, [([3], 17)]), device="cpu", num_blocks=8)
    # a block past the keys a row reads is not checked (tables may be padded)
    sea.build_paged_batch_metadata(_step(sea, [([3, 99], 16)]), device="cpu", num_blocks=8)
    sea.build_paged_batch_metadata(_step(sea, [([3, 99], 20)]), device="cpu")


def test_copy_blocks_checks_host_ids():
    import pytest
    import torch

    sea = sea_module()
    cache = sea._PagedKVCache(torch.zeros(1, 2, 8, 16, 1, 8))
    with pytest.raises(ValueError, match="also a source"):
        cache.copy_blocks([1, 2], [2, 3])
    with pytest.raises(ValueError, match="unique"):
        cache.copy_blocks([1, 2], [4, 4])
    with pytest.raises(IndexError):
        cache.copy_blocks([1], [8])
    with pytest.raises(IndexError):
        cache.copy_blocks([-1], [3])
