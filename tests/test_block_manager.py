"""Block manager (serving-engine_amd/block_manager.py): the behaviours the
reference's tests/test_block_manager.py pins for
serving_engine/block_manager.py -- pool accounting, block tables, ref counts,
chained-hash prefix matching, preemption -- and copy-on-write of shared
blocks, which the reference does not have."""
import importlib

import pytest

bmm = importlib.import_module("serving-engine_amd.block_manager")
reqm = importlib.import_module("serving-engine_amd.request")
BlockManager = bmm.BlockManager
Request, RequestPhase, RequestStatus = reqm.Request, reqm.RequestPhase, reqm.RequestStatus


def req(rid, n, tokens=None):
    return Request(request_id=rid, prompt_token_ids=list(tokens if tokens is not None else range(n)))


def computed(bm, r, n):
    r.num_computed_tokens = n
    bm.register_computed_blocks(r)


# -- pool and tables ----------------------------------------------------------

def test_allocation_is_ceil_of_length_over_block_size():
    bm = BlockManager(10)
    for n, want in ((1, 1), (16, 1), (17, 2), (20, 2), (48, 3)):
        r = req("a", n)
        assert bm.can_allocate(r)
        bm.allocate(r)
        assert len(r.block_table) == want
        bm.free(r)
    assert bm.get_num_free_blocks() == 10


def test_allocation_refused_beyond_the_pool():
    bm = BlockManager(1)
    assert not bm.can_allocate(req("a", 20))
    assert bm.can_allocate(req("b", 16))


def test_ids_come_from_the_top_of_the_pool():
    bm = BlockManager(6)
    r = req("a", 40)
    bm.allocate(r)
    assert r.block_table == [5, 4, 3]
    assert all(bm.blocks[b].ref_count == 1 for b in r.block_table)


def test_allocation_covers_generated_tokens_too():
    bm = BlockManager(10)
    r = req("a", 16)
    r.output_token_ids = [7] * 5  # a preempted request recomputes its outputs as well
    bm.allocate(r)
    assert len(r.block_table) == 2


def test_append_slot_grows_only_a_full_table():
    bm = BlockManager(10)
    r = req("a", 20)
    bm.allocate(r)  # 2 blocks, room for 32 tokens
    r.output_token_ids = [1]
    assert bm.append_slot(r) is None and len(r.block_table) == 2
    r.output_token_ids = [1] * 13  # total 33
    new = bm.append_slot(r)
    assert new == r.block_table[-1] and len(r.block_table) == 3
    assert bm.get_num_free_blocks() == 7


def test_block_boundary_admission_has_room_for_the_next_token():
    bm = BlockManager(10)
    r = req("a", 16)
    bm.allocate(r)
    r.output_token_ids = [1]  # position 16: a second block
    assert bm.can_append_slot(r)
    bm.append_slot(r)
    assert len(r.block_table) == 2


def test_free_returns_blocks_and_empties_the_table():
    bm = BlockManager(10)
    r = req("a", 32)
    bm.allocate(r)
    assert bm.get_num_free_blocks() == 8
    bm.free(r)
    assert bm.get_num_free_blocks() == 10 and r.block_table == []
    for _ in range(50):  # repeated cycles never leak
        bm.allocate(r)
        bm.free(r)
    assert bm.get_num_free_blocks() == 10


def test_fork_shares_blocks_with_an_independent_table():
    bm = BlockManager(10)
    parent, child = req("p", 32), req("c", 32)
    bm.allocate(parent)
    bm.fork(parent, child)
    assert child.block_table == parent.block_table and child.block_table is not parent.block_table
    assert all(bm.blocks[b].ref_count == 2 for b in parent.block_table)
    child.block_table.append(99)
    assert 99 not in parent.block_table
    child.block_table.pop()
    bm.free(parent)
    assert bm.get_num_free_blocks() == 8  # still held by the child
    bm.free(child)
    assert bm.get_num_free_blocks() == 10


def test_preempt_frees_and_resets_for_recompute():
    bm = BlockManager(10)
    r = req("a", 40)
    bm.allocate(r)
    r.num_computed_tokens, r.phase, r.status = 40, RequestPhase.NEEDS_DECODE, RequestStatus.RUNNING
    r.output_token_ids = [3, 4]
    bm.preempt(r)
    assert bm.get_num_free_blocks() == 10 and r.block_table == []
    assert r.num_computed_tokens == 0 and r.phase == RequestPhase.NEEDS_PREFILL
    assert r.status == RequestStatus.PREEMPTED and r.output_token_ids == [3, 4]


# -- prefix matching ----------------------------------------------------------

def test_no_match_in_an_empty_index():
    bm = BlockManager(10)
    r = req("a", 32)
    bm.match_prefix(r)
    assert r.block_table == [] and r.num_computed_tokens == 0


def test_registered_blocks_are_matched_and_shared():
    bm = BlockManager(10)
    a = req("a", 40)
    bm.allocate(a)
    computed(bm, a, 40)
    b = req("b", 40)
    bm.match_prefix(b)
    assert b.block_table == a.block_table[:2]  # the partial third block is never registered
    assert b.num_computed_tokens == 32
    assert [bm.blocks[x].ref_count for x in b.block_table] == [2, 2]


def test_matching_stops_at_the_first_different_block():
    bm = BlockManager(10)
    a = req("a", 48)
    bm.allocate(a)
    computed(bm, a, 48)
    toks = list(range(48))
    toks[20] = -1  # second block differs; the third is identical but its chain is not
    b = req("b", 48, toks)
    bm.match_prefix(b)
    assert b.block_table == a.block_table[:1] and b.num_computed_tokens == 16


def test_a_block_is_keyed_by_everything_before_it():
    bm = BlockManager(10)
    a = req("a", 32, [1] * 16 + [2] * 16)
    bm.allocate(a)
    computed(bm, a, 32)
    b = req("b", 32, [3] * 16 + [2] * 16)  # same second block, other history
    bm.match_prefix(b)
    assert b.block_table == []


def test_registration_in_chunks_equals_registration_at_once():
    one, two = BlockManager(10), BlockManager(10)
    a, b = req("a", 48), req("b", 48)
    one.allocate(a)
    computed(one, a, 48)
    two.allocate(b)
    for n in (16, 20, 48):
        computed(two, b, n)
    assert [one.blocks[x].content_hash for x in a.block_table] == \
        [two.blocks[x].content_hash for x in b.block_table]


def test_only_computed_prompt_blocks_are_registered():
    bm = BlockManager(10)
    r = req("a", 32)
    bm.allocate(r)
    computed(bm, r, 20)
    assert bm.blocks[r.block_table[0]].content_hash is not None
    assert bm.blocks[r.block_table[1]].content_hash is None
    assert len(bm.hash_to_block) == 1
    r.output_token_ids = list(range(40))  # generated tokens never enter the index
    computed(bm, r, 72)
    assert len(bm.hash_to_block) == 2


def test_first_registered_block_stays_canonical():
    bm = BlockManager(10)
    a, b = req("a", 16), req("b", 16)  # same content, both missed the index
    bm.allocate(a)
    bm.allocate(b)
    assert a.block_table != b.block_table
    computed(bm, a, 16)
    computed(bm, b, 16)
    assert bm.hash_to_block == {bm.blocks[a.block_table[0]].content_hash: a.block_table[0]}
    assert bm.blocks[b.block_table[0]].content_hash is None
    bm.free(b)
    assert len(bm.hash_to_block) == 1
    bm.free(a)
    assert bm.hash_to_block == {}


def test_freed_block_leaves_the_index_only_with_its_last_holder():
    bm = BlockManager(10)
    a = req("a", 16)
    bm.allocate(a)
    computed(bm, a, 16)
    b = req("b", 16)
    bm.match_prefix(b)
    bm.free(a)
    assert len(bm.hash_to_block) == 1  # b still holds it
    c = req("c", 16)
    bm.match_prefix(c)
    assert c.block_table == b.block_table
    bm.free(b)
    bm.free(c)
    assert bm.hash_to_block == {} and bm.get_num_free_blocks() == 10
    d = req("d", 16)
    bm.match_prefix(d)
    assert d.block_table == []


def test_allocation_counts_matched_blocks_as_held():
    bm = BlockManager(3)
    a = req("a", 32)
    bm.allocate(a)
    computed(bm, a, 32)
    b = req("b", 48)
    bm.match_prefix(b)  # 2 blocks matched, 1 missing, 1 free
    assert bm.can_allocate(b)
    bm.allocate(b)
    assert b.block_table[:2] == a.block_table and bm.get_num_free_blocks() == 0


# -- copy-on-write -------------------------------------------------------------

def test_writing_into_a_shared_partial_block_copies_it():
    bm = BlockManager(10)
    parent = req("p", 20)
    bm.allocate(parent)  # [9, 8]; block 8 holds tokens 16..19 of 32
    child = req("c", 20)
    bm.fork(parent, child)
    child.output_token_ids = [5]  # position 20: in shared block 8
    assert bm.can_append_slot(child)
    new = bm.append_slot(child)
    assert child.block_table == [9, new] and new not in (8, 9)
    assert parent.block_table == [9, 8]
    assert bm.take_copies() == [(8, new)] and bm.take_copies() == []
    assert (bm.blocks[8].ref_count, bm.blocks[9].ref_count, bm.blocks[new].ref_count) == (1, 2, 1)
    parent.output_token_ids = [6]  # block 8 is the parent's alone now: written in place
    assert bm.append_slot(parent) is None and bm.take_copies() == []


def test_shared_full_blocks_are_not_copied():
    bm = BlockManager(10)
    parent = req("p", 32)
    bm.allocate(parent)
    child = req("c", 32)
    bm.fork(parent, child)
    child.output_token_ids = [1]  # position 32: a new block of its own
    bm.append_slot(child)
    assert bm.take_copies() == [] and child.block_table[:2] == parent.block_table


def test_copy_needs_a_free_block():
    bm = BlockManager(2)
    parent = req("p", 20)
    bm.allocate(parent)
    child = req("c", 20)
    bm.fork(parent, child)
    child.output_token_ids = [1]
    assert not bm.can_append_slot(child)
    parent.output_token_ids = [1]
    assert not bm.can_append_slot(parent)


def test_prepare_write_copies_each_shared_block_of_a_range():
    bm = BlockManager(10)
    a = req("a", 40)
    bm.allocate(a)
    b = req("b", 40)
    bm.fork(a, b)
    assert bm.shared_blocks_in(b, 10, 40) == 3
    pairs = bm.prepare_write(b, 10, 34)
    assert [s for s, _ in pairs] == a.block_table
    assert [d for _, d in pairs] == b.block_table
    assert bm.shared_blocks_in(b, 0, 48) == 0 and bm.shared_blocks_in(a, 0, 48) == 0
    assert bm.get_num_free_blocks() == 4


def test_bad_pool_sizes_are_rejected():
    with pytest.raises(ValueError):
        BlockManager(-1)
    with pytest.raises(ValueError):
        BlockManager(4, block_size=0)
