"""Scheduler (serving-engine_amd/scheduler.py): the behaviours the reference's
tests/test_scheduler.py pins for serving_engine/scheduler.py -- admission,
running-before-waiting, LIFO eviction only on a true stall, the sequence and
token caps, finishing, prefix-cache reuse -- plus chunked prefill, the
step's copy-on-write pairs and a randomized run that checks the pool's
accounting after every step."""
import importlib
import random

bmm = importlib.import_module("serving-engine_amd.block_manager")
reqm = importlib.import_module("serving-engine_amd.request")
schm = importlib.import_module("serving-engine_amd.scheduler")
BlockManager, Scheduler = bmm.BlockManager, schm.Scheduler
Request, RequestPhase, RequestStatus = reqm.Request, reqm.RequestPhase, reqm.RequestStatus


def req(rid, n, max_new=256, eos=None):
    return Request(request_id=rid, prompt_token_ids=list(range(n)), max_new_tokens=max_new, eos_token_id=eos)


def sched(blocks, bs=4, **kw):
    return Scheduler(BlockManager(blocks, block_size=bs), **kw)


def running_decode(s, r, allocate=True):
    """Puts r in the running set as a decode row (optionally with blocks)."""
    if allocate:
        s.block_manager.allocate(r)
    r.phase, r.status = RequestPhase.NEEDS_DECODE, RequestStatus.RUNNING
    s.running.append(r)
    return r


def test_new_requests_wait():
    s = sched(10)
    r = req("a", 5)
    s.add_request(r)
    assert s.waiting == [r] and s.running == [] and r.status == RequestStatus.WAITING


def test_admission_allocates_and_runs_the_whole_prompt():
    s = sched(10)
    r = req("a", 6)
    s.add_request(r)
    out = s.schedule()
    assert out.scheduled_requests == [r] and out.prefill_chunk_sizes == {"a": 6}
    assert out.prefill_final_chunk == {"a"} and r.status == RequestStatus.RUNNING
    assert s.running == [r] and s.waiting == [] and len(r.block_table) == 2


def test_no_admission_without_blocks_for_the_prompt():
    s = sched(1)
    r = req("a", 6)
    s.add_request(r)
    out = s.schedule()
    assert out.scheduled_requests == [] and s.waiting == [r] and r.block_table == []


def test_decode_with_room_takes_no_block():
    s = sched(10)
    r = running_decode(s, req("a", 5))
    r.output_token_ids = [1]
    free = s.block_manager.get_num_free_blocks()
    assert s.schedule().scheduled_requests == [r]
    assert s.block_manager.get_num_free_blocks() == free


def test_blocked_decode_waits_while_others_progress():
    s = sched(1)
    blocked = req("blocked", 3)
    s.add_request(blocked)
    s.schedule()  # takes the only block
    blocked.phase, blocked.output_token_ids = RequestPhase.NEEDS_DECODE, [1, 2]  # needs a second block
    other = running_decode(s, req("other", 3), allocate=False)
    other.block_table, other.output_token_ids = [0], [1]  # fits its block
    out = s.schedule()
    assert out.scheduled_requests == [other] and out.preempted_requests == []


def test_running_rows_come_before_waiting_ones():
    s = sched(1)
    r = running_decode(s, req("r", 4), allocate=False)  # needs the one free block
    w = req("w", 4)
    s.add_request(w)
    out = s.schedule()
    assert out.scheduled_requests == [r] and s.waiting == [w]


def test_true_stall_evicts_the_latest_admitted():
    s = sched(2)
    first = running_decode(s, req("first", 4))
    last = running_decode(s, req("last", 4))
    first.output_token_ids = last.output_token_ids = [1, 2, 3, 4]  # both need a block; none free
    out = s.schedule()
    assert out.scheduled_requests == [first] and len(first.block_table) == 2
    assert out.preempted_requests == [last] and last not in s.running and last in s.waiting
    assert last.block_table == [] and last.phase == RequestPhase.NEEDS_PREFILL
    assert last.status == RequestStatus.PREEMPTED


def test_stall_without_a_victim_schedules_nothing():
    s = sched(1)
    only = running_decode(s, req("only", 4))
    only.output_token_ids = [1, 2, 3, 4]
    out = s.schedule()
    assert out.scheduled_requests == [] and out.preempted_requests == [] and s.running == [only]


def test_prefill_step_advances_and_turns_to_decode():
    s = sched(10)
    r = req("a", 6)
    s.add_request(r)
    out = s.schedule()
    r.output_token_ids = [9]
    s.update_after_step(out)
    assert r.num_computed_tokens == 6 and r.phase == RequestPhase.NEEDS_DECODE
    assert r.status == RequestStatus.RUNNING


def test_finishing_on_max_new_tokens_frees_blocks():
    s = sched(10)
    r = req("a", 4, max_new=2)
    s.add_request(r)
    s.update_after_step(s.schedule())
    r.output_token_ids = [5, 6]
    s.update_after_step(s.schedule())
    assert r.status == RequestStatus.FINISHED and r.block_table == [] and s.running == []
    assert s.block_manager.get_num_free_blocks() == 10


def test_eos_finishes_at_prefill_and_at_decode():
    for at_prefill in (True, False):
        s = sched(10)
        r = req("a", 4, eos=42)
        s.add_request(r)
        out = s.schedule()
        if at_prefill:
            r.output_token_ids = [42]
        else:
            r.output_token_ids = [7]
            s.update_after_step(out)
            out = s.schedule()
            r.output_token_ids.append(42)
        s.update_after_step(out)
        assert r.status == RequestStatus.FINISHED and not s.has_unfinished_requests()


def test_sequence_cap():
    s = sched(10, max_num_seqs=2)
    rs = [req(f"r{i}", 3) for i in range(3)]
    for r in rs:
        s.add_request(r)
    out = s.schedule()
    assert out.scheduled_requests == rs[:2] and s.waiting == [rs[2]]


def test_token_cap_stops_piling_on():
    s = sched(10, max_num_batched_tokens=5)
    a, b = req("a", 4), req("b", 4)
    s.add_request(a)
    s.add_request(b)
    out = s.schedule()
    assert out.scheduled_requests == [a] and s.waiting == [b]


def test_lone_candidate_over_the_cap_still_runs():
    s = sched(10, max_num_batched_tokens=3)
    r = req("a", 8)
    s.add_request(r)
    out = s.schedule()
    assert out.scheduled_requests == [r]
    assert out.prefill_chunk_sizes["a"] == 3 and out.prefill_final_chunk == set()  # a first chunk


def test_decode_spends_a_tight_budget_first():
    s = sched(10, max_num_batched_tokens=1)
    r = running_decode(s, req("r", 4))
    r.output_token_ids = [1]
    w = req("w", 4)
    s.add_request(w)
    assert s.schedule().scheduled_requests == [r] and s.waiting == [w]


def test_budget_skip_is_not_a_stall():
    s = sched(10, max_num_batched_tokens=1)
    a = running_decode(s, req("a", 1))
    b = running_decode(s, req("b", 1))
    a.output_token_ids = b.output_token_ids = [1]
    out = s.schedule()
    assert out.scheduled_requests == [a] and out.preempted_requests == [] and b in s.running


def test_unfinished_until_the_last_request_ends():
    s = sched(10)
    r = req("a", 4, max_new=1)
    s.add_request(r)
    assert s.has_unfinished_requests()
    out = s.schedule()
    r.output_token_ids = [1]
    assert s.has_unfinished_requests()
    s.update_after_step(out)
    assert not s.has_unfinished_requests()


def test_cached_prompt_is_admitted_with_nothing_to_compute():
    s = sched(10)
    a = req("a", 4)
    s.add_request(a)
    s.update_after_step(s.schedule())  # a's block enters the prefix index
    b = req("b", 4)
    s.add_request(b)
    assert b.num_computed_tokens == 4 and b.block_table == a.block_table
    out = s.schedule()
    assert b in out.scheduled_requests and out.prefill_chunk_sizes["b"] == 0
    assert "b" in out.prefill_final_chunk
    assert s.block_manager.blocks[a.block_table[0]].ref_count == 2


def test_chunked_prefill_fills_the_budget_past_the_floor():
    s = sched(20, max_num_batched_tokens=8, min_chunk_size=2)
    a, b = req("a", 6), req("b", 10)
    s.add_request(a)
    s.add_request(b)
    out = s.schedule()
    assert out.prefill_chunk_sizes == {"a": 6, "b": 2} and out.prefill_final_chunk == {"a"}
    a.output_token_ids = [1]
    s.update_after_step(out)
    assert b.num_computed_tokens == 2 and b.phase == RequestPhase.NEEDS_PREFILL
    out = s.schedule()  # a decodes (1 token), b continues with the other 7
    assert out.scheduled_requests == [a, b] and out.prefill_chunk_sizes == {"b": 7}


def test_forked_decode_rows_get_copies_of_their_shared_block():
    s = sched(10)
    parent = running_decode(s, req("p", 6))  # blocks [9, 8]; 8 holds tokens 4..5 of 8
    child = req("c", 6)
    s.block_manager.fork(parent, child)
    running_decode(s, child, allocate=False)
    parent.output_token_ids = [1]
    child.output_token_ids = [2]  # both write position 6, in block 8
    out = s.schedule()
    assert out.scheduled_requests == [parent, child]
    (src, dst), = out.blocks_to_copy  # the parent copied first; the child then held 8 alone
    assert src == 8 and parent.block_table == [9, dst] and child.block_table == [9, 8]
    assert s.schedule().blocks_to_copy == []


def test_randomized_run_keeps_the_pool_consistent():
    rng = random.Random(7)
    bs, nblocks = 4, 24
    s = sched(nblocks, bs=bs, max_num_batched_tokens=24, max_num_seqs=6, min_chunk_size=3)
    pending = [req(f"r{i}", rng.randint(1, 20), max_new=rng.randint(1, 12)) for i in range(30)]
    steps = 0
    while pending or s.has_unfinished_requests():
        if pending and rng.random() < 0.5:
            s.add_request(pending.pop())
        out = s.schedule()
        for r in out.scheduled_requests:
            end = r.total_len if r.phase == RequestPhase.NEEDS_DECODE else \
                r.num_computed_tokens + out.prefill_chunk_sizes[r.request_id]
            assert len(r.block_table) * bs >= end  # room for every token the step writes
            if r.phase == RequestPhase.NEEDS_DECODE or r.request_id in out.prefill_final_chunk:
                r.output_token_ids.append(rng.randint(0, 99))
        s.update_after_step(out)
        held = {}
        for r in s.running + s.waiting:  # a waiting request may hold prefix-matched blocks
            for b in r.block_table:
                held[b] = held.get(b, 0) + 1
        bm = s.block_manager
        assert all(bm.blocks[b].ref_count == held.get(b, 0) for b in range(nblocks))
        assert sorted(bm.free_blocks) == [b for b in range(nblocks) if b not in held]
        steps += 1
        assert steps < 2000
    assert s.block_manager.get_num_free_blocks() == nblocks


def test_randomized_run_with_forks_keeps_copies_and_accounting_consistent():
    rng = random.Random(11)
    bs, nblocks = 4, 40
    s = sched(nblocks, bs=bs, max_num_batched_tokens=20, max_num_seqs=8, min_chunk_size=2)
    pending = [req(f"r{i}", rng.randint(2, 18), max_new=rng.randint(2, 10)) for i in range(24)]
    nfork = copies = 0
    for step in range(3000):
        if not pending and not s.has_unfinished_requests():
            break
        if pending and rng.random() < 0.4:
            s.add_request(pending.pop())
        decoding = [r for r in s.running if r.phase == RequestPhase.NEEDS_DECODE and r.block_table]
        if decoding and rng.random() < 0.3 and s.block_manager.get_num_free_blocks() > 2:
            p = rng.choice(decoding)
            c = Request(request_id=f"f{nfork}", prompt_token_ids=list(p.prompt_token_ids),
                        output_token_ids=list(p.output_token_ids), max_new_tokens=p.max_new_tokens)
            c.num_computed_tokens, c.phase, c.status = p.num_computed_tokens, p.phase, RequestStatus.RUNNING
            s.block_manager.fork(p, c)
            s.running.append(c)
            nfork += 1
        held_before = {b for r in s.running + s.waiting for b in r.block_table}
        free_before = set(s.block_manager.free_blocks)
        out = s.schedule()
        for src, dst in out.blocks_to_copy:
            assert src in held_before and dst in free_before and src != dst
            assert any(dst in r.block_table for r in out.scheduled_requests)
        assert len({d for _, d in out.blocks_to_copy}) == len(out.blocks_to_copy)
        copies += len(out.blocks_to_copy)
        for r in out.scheduled_requests:
            if r.phase == RequestPhase.NEEDS_DECODE:
                i = (r.total_len - 1) // bs  # the block this step writes is this row's alone
                assert s.block_manager.blocks[r.block_table[i]].ref_count == 1
            if r.phase == RequestPhase.NEEDS_DECODE or r.request_id in out.prefill_final_chunk:
                r.output_token_ids.append(rng.randint(0, 99))
        s.update_after_step(out)
        held = {}
        for r in s.running + s.waiting:  # a waiting request may hold prefix-matched blocks
            for b in r.block_table:
                held[b] = held.get(b, 0) + 1
        bm = s.block_manager
        assert all(bm.blocks[b].ref_count == held.get(b, 0) for b in range(nblocks))
        assert sorted(bm.free_blocks) == [b for b in range(nblocks) if b not in held]
    assert not pending and not s.has_unfinished_requests()
    assert nfork > 0 and copies > 0
    assert s.block_manager.get_num_free_blocks() == nblocks
