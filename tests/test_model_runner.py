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
