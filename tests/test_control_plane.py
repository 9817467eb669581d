"""CPU tests of the kvflux::v2 control plane through the Python binding.

Each test restates the assertions of one of the reference's CPU tests
(file:line given per test) so the known-answer page ids, slots and tables
are pinned here as well as by the compiled reference tests in
test_reference_compat.py.
"""
from __future__ import annotations

import pytest


def occupy_until(pool, occupied, next_id):
    while pool.capacity() - pool.available() < next_id:
        occupied.append(pool.allocate())


def test_physical_block_pool_reuse_refs_capacity(v2):
    # reference tests/physical_block_pool_test.cpp:18-72
    with pytest.raises(ValueError):
        v2.PhysicalBlockPool(0, 16)
    with pytest.raises(ValueError):
        v2.PhysicalBlockPool(1024, 0)
    pool = v2.PhysicalBlockPool(1024, 16)
    assert (pool.capacity(), pool.block_size(), pool.available()) == (1024, 16, 1024)
    first, middle, third = pool.allocate(), pool.allocate(), pool.allocate()
    assert [pool.id(h) for h in (first, middle, third)] == [0, 1, 2]
    pool.free(middle)
    reused = pool.allocate()
    assert pool.id(reused) == middle.id and reused.generation != middle.generation
    with pytest.raises(ValueError):
        pool.id(middle)
    with pytest.raises(ValueError):
        pool.free(middle)
    pool.retain(first)
    assert pool.ref_count(first) == 2
    pool.free(first)
    assert pool.ref_count(first) == 1 and pool.available() == 1021
    rest = [pool.allocate() for _ in range(1021)]
    assert [pool.id(h) for h in rest] == list(range(3, 1024))
    with pytest.raises(v2.CapacityError):
        pool.allocate()
    with pytest.raises(ValueError):
        pool.id(v2.PhysicalBlockHandle(1024, 1))
    pool.free(first)
    again = pool.allocate()
    assert pool.id(again) == first.id and again.generation != first.generation
    with pytest.raises(ValueError):
        pool.retain(first)
    for h in [again, reused, third, *rest]:
        pool.free(h)
    assert pool.available() == pool.capacity()


def test_block_table_exact_mapping_and_sharing(v2):
    # reference tests/block_table_test.cpp:26-59
    pool = v2.PhysicalBlockPool(100, 16)
    initial = [pool.allocate() for _ in range(92)]
    a = v2.BlockTable(pool)
    for physical in (27, 91, 3, 48):
        a.append_existing(initial[physical])
    assert [a.physical_id(i) for i in range(4)] == [27, 91, 3, 48] and a[0] == 27
    with pytest.raises(IndexError):
        a.physical_id(4)
    for h in initial:
        pool.free(h)
    assert pool.available() == 96
    b = v2.BlockTable(pool)
    b.append_shared(a, 1)
    b.append_shared(a, 3)
    assert (b.physical_id(0), b.physical_id(1)) == (91, 48) and pool.available() == 96
    a.pop_back()
    assert len(a) == 3 and b.physical_id(1) == 48
    a.clear()
    assert a.empty() and pool.available() == 98
    b.clear()
    assert pool.available() == pool.capacity()
    with pytest.raises(IndexError):
        b.pop_back()


def test_block_table_capacity_and_move(v2):
    # reference tests/block_table_test.cpp:61-83
    pool = v2.PhysicalBlockPool(2, 16)
    a = v2.BlockTable(pool)
    assert a.append_new() == 0 and a.append_new() == 1
    with pytest.raises(v2.CapacityError):
        a.append_new()
    moved = v2.BlockTable.moved(a)
    assert a.empty() and moved.physical_id(0) == 0
    with pytest.raises(v2.LogicError):
        a.append_new()
    moved.append_shared(moved, 0)
    assert len(moved) == 3 and pool.available() == 0
    dest = v2.BlockTable(pool)
    dest.move_from(moved)
    assert moved.empty() and len(dest) == 3
    dest.pop_back()
    assert pool.available() == 0
    dest.clear()
    assert pool.available() == 2


def test_block_table_invalid_inputs_do_not_mutate(v2):
    # reference tests/block_table_test.cpp:85-98
    pool, other_pool = v2.PhysicalBlockPool(2, 16), v2.PhysicalBlockPool(2, 16)
    a, other = v2.BlockTable(pool), v2.BlockTable(other_pool)
    stale = pool.allocate()
    pool.free(stale)
    with pytest.raises(ValueError):
        a.append_existing(stale)
    assert a.empty() and pool.available() == 2
    a.append_new()
    with pytest.raises(IndexError):
        a.append_shared(a, 1)
    with pytest.raises(ValueError):
        a.append_shared(other, 0)
    assert len(a) == 1 and pool.available() == 1


def test_sequence_state_virtual_blocks(v2):
    # reference tests/sequence_state_test.cpp:27-62
    pool = v2.PhysicalBlockPool(100, 16)
    occupied = []
    request = v2.SequenceState(1001, pool)
    assert (request.request_id(), request.block_size(), request.num_tokens()) == (1001, 16, 0)
    assert request.last_block_num_tokens() == 0

    def until(n):
        while len(occupied) < n:
            occupied.append(pool.allocate())

    until(7); request.append_tokens(16)
    until(32); request.append_tokens(16)
    until(89); request.append_tokens(3)
    assert request.num_tokens() == 35 and request.num_allocated_blocks() == 3
    assert request.last_block_num_tokens() == 3
    assert [request.physical_block_id(i) for i in range(3)] == [7, 33, 91]
    loc = request.token_location(34)
    assert (loc.physical_block, loc.offset_in_block) == (91, 2)
    with pytest.raises(IndexError):
        request.token_location(35)
    with pytest.raises(IndexError):
        request.physical_block_id(3)
    for h in occupied:
        pool.free(h)
    assert pool.available() == 97


def test_sequence_state_tail_growth_and_rollback(v2):
    # reference tests/sequence_state_test.cpp:99-126
    pool = v2.PhysicalBlockPool(2, 16)
    request = v2.SequenceState(42, pool)
    request.append_tokens(15)
    request.append_tokens(1)
    assert request.num_allocated_blocks() == 1 and request.last_block_num_tokens() == 16
    request.append_tokens(0)
    with pytest.raises(v2.CapacityError):
        request.append_tokens(32)
    assert request.num_tokens() == 16 and request.num_allocated_blocks() == 1
    assert pool.available() == 1
    with pytest.raises(OverflowError):
        request.append_tokens(2**64 - 1)
    seventeenth = request.append_token()
    assert (seventeenth.physical_block, seventeenth.offset_in_block) == (1, 0)
    request.append_tokens(15)
    with pytest.raises(v2.CapacityError):
        request.append_token()
    assert request.num_tokens() == 32


def test_sequence_move_returns_previous_pages(v2):
    # reference tests/sequence_state_test.cpp:128-143
    first_pool, second_pool = v2.PhysicalBlockPool(2, 16), v2.PhysicalBlockPool(1, 8)
    first = v2.SequenceState(1001, first_pool)
    first.append_tokens(17)
    second = v2.SequenceState(2002, second_pool)
    second.append_tokens(1)
    second.move_from(first)
    assert second_pool.available() == 1
    assert first.num_tokens() == 0 and first.num_allocated_blocks() == 0
    assert (second.request_id(), second.num_tokens(), second.block_size()) == (1001, 17, 16)
    assert first_pool.available() == 0
    del second, first
    assert first_pool.available() == 2 and second_pool.available() == 1


def test_slot_mapping_known_answers(v2):
    # reference tests/slot_mapping_test.cpp:26-62
    pool = v2.PhysicalBlockPool(160, 16)
    occupied = []
    occupy_until(pool, occupied, 31)
    b = v2.SequenceState(1002, pool); b.append_tokens(18)
    occupy_until(pool, occupied, 79)
    a = v2.SequenceState(1001, pool); a.append_tokens(35)
    occupy_until(pool, occupied, 133)
    c = v2.SequenceState(1003, pool); c.append_tokens(81)
    assert v2.build_slot_mapping([(a, 34), (b, 17), (c, 80)]) == [1298, 513, 2208]
    c.append_tokens(8)
    assert v2.build_slot_mapping([(c, 88)]) == [2216]


def test_slot_mapping_rejects_invalid_batches(v2):
    # reference tests/slot_mapping_test.cpp:64-79
    p1, p2 = v2.PhysicalBlockPool(2, 16), v2.PhysicalBlockPool(2, 16)
    first, second = v2.SequenceState(1, p1), v2.SequenceState(2, p2)
    first.append_tokens(16); second.append_tokens(1)
    assert v2.build_slot_mapping([]) == []
    assert v2.build_slot_mapping([(first, 15), (first, 0)]) == [15, 0]
    with pytest.raises(ValueError):
        v2.build_slot_mapping([(None, 0)])
    with pytest.raises(ValueError):
        v2.build_slot_mapping([(first, 0), (None, 0)])
    with pytest.raises(IndexError):
        v2.build_slot_mapping([(first, 16)])
    with pytest.raises(ValueError):
        v2.build_slot_mapping([(first, 0), (second, 0)])
    assert first.num_tokens() == 16 and p1.available() == 1 and p2.available() == 1


def test_batch_block_table_padded_rows(v2):
    # reference tests/batch_block_table_test.cpp:18-44
    assert v2.build_batch_block_table([]).num_sequences() == 0
    pool = v2.PhysicalBlockPool(16, 16)
    a, b, c, e = (v2.SequenceState(i, pool) for i in (1, 2, 3, 4))
    for s, n in ((a, 16), (b, 16), (c, 16), (a, 16), (b, 16), (c, 12), (a, 3), (b, 29)):
        s.append_tokens(n)
    t = v2.build_batch_block_table([a, b, c, e])
    pad = v2.BatchBlockTable.invalid_block()
    assert t.num_sequences() == 4 and t.max_blocks_per_sequence() == 4
    assert t.sequence_lengths() == [35, 61, 28, 0]
    assert t.block_table() == [0, 3, 6, pad, 1, 4, 7, 8, 2, 5, pad, pad, pad, pad, pad, pad]
    assert t.physical_id(1, 3) == 8 and t.physical_id(2, 1) == 5
    for r, blk in ((0, 3), (3, 0), (4, 0)):
        with pytest.raises(IndexError):
            t.physical_id(r, blk)
    with pytest.raises(ValueError):
        v2.build_batch_block_table([a, None])
    other = v2.SequenceState(5, v2.PhysicalBlockPool(2, 16))
    with pytest.raises(ValueError):
        v2.build_batch_block_table([a, other])


def test_read_block_table_27_3_91(v2):
    # reference tests/paged_kv_read_table_test.cpp:12-31
    pool = v2.PhysicalBlockPool(96, 16)
    occupied = [pool.allocate() for _ in range(27)]
    request = v2.SequenceState(1001, pool)
    assert v2.build_read_block_table(request) == []
    request.append_tokens(16)
    occupied += [pool.allocate() for _ in range(28, 91)]
    pool.free(occupied[3])
    request.append_tokens(16)
    request.append_tokens(8)
    assert request.num_tokens() == 40 and request.last_block_num_tokens() == 8
    assert v2.build_read_block_table(request) == [27, 3, 91]


@pytest.mark.parametrize("dtype,esize", [("Float16", 2), ("BFloat16", 2), ("Float32", 4)])
def test_paged_kv_layout_dense_enumeration(v2, dtype, esize):
    # reference tests/paged_kv_layout_test.cpp:17-51
    layout = v2.PagedKVLayout(3, 2, 4, 3, getattr(v2.DType, dtype))
    assert layout.page_bytes() == 2 * 4 * 3 * esize
    assert layout.total_bytes() == 2 * layout.cache_bytes() and layout.slot_count() == 12
    expected = 0
    for kind in (v2.KVKind.Key, v2.KVKind.Value):
        for block in range(3):
            assert layout.page_byte_offset(kind, block) == expected
            for head in range(2):
                for token in range(4):
                    for dim in range(3):
                        assert layout.byte_offset(kind, block, head, token, dim) == expected
                        assert layout.slot_byte_offset(kind, block * 4 + token, head, dim) == expected
                        expected += esize
    assert expected == layout.total_bytes()
    for args in ((v2.KVKind.Key, 0, 2, 0, 0), (v2.KVKind.Key, 0, 0, 4, 0), (v2.KVKind.Key, 0, 0, 0, 3)):
        with pytest.raises(IndexError):
            layout.byte_offset(*args)
    with pytest.raises(IndexError):
        layout.slot_byte_offset(v2.KVKind.Key, 12, 0, 0)
    with pytest.raises(ValueError):
        v2.PagedKVLayout(0, 1, 1, 1, v2.DType.Float16)
    with pytest.raises(OverflowError):
        v2.PagedKVLayout(2**64 - 1, 1, 1, 1, v2.DType.Float16)


def test_fragmented_odd_pages_and_exhaustion(v2):
    # reference tests/fragmentation_test.cpp:9-40
    pool = v2.PhysicalBlockPool(128, 4)
    holders = [pool.allocate() for _ in range(128)]
    for nxt in range(128, 0, -2):
        pool.free(holders[nxt - 1])
    assert pool.available() == 64
    request = v2.SequenceState(2001, pool)
    request.append_tokens(64 * 4)
    assert v2.build_read_block_table(request) == list(range(1, 128, 2))
    with pytest.raises(v2.CapacityError):
        request.append_token()
    assert request.num_tokens() == 256
    del request
    assert pool.available() == 64


def test_copy_on_write_of_shared_partial_tail(v2):
    # reference tests/copy_on_write_test.cpp:21-58 (CPU page copier)
    pool = v2.PhysicalBlockPool(3, 4)
    pages = [[0] * 4 for _ in range(3)]
    a = v2.SequenceState(1, pool)
    a.append_tokens(3)
    old = a.physical_block_id(0)
    pages[old] = [11, 22, 33, -1]
    b = a.fork_shared(2)
    assert b.num_tokens() == 3 and pool.ref_count(a.block_table().handle(0)) == 2
    with pytest.raises(v2.LogicError):
        a.append_token()
    copies = []

    def copier(src, dst):
        copies.append((src.id, dst.id))
        pages[dst.id] = list(pages[src.id])

    loc = a.append_token_with_copy(copier)
    assert len(copies) == 1 and loc.physical_block != old and loc.offset_in_block == 3
    assert pages[loc.physical_block] == [11, 22, 33, -1]
    assert b.physical_block_id(0) == old and pool.ref_count(b.block_table().handle(0)) == 1
    b_loc = b.append_token()
    assert b_loc.physical_block == old and b_loc.offset_in_block == 3


def test_prefix_cache_shares_full_blocks(v2):
    # reference tests/paged_kv_read_test.cpp:92-106 (metadata part)
    pool = v2.PhysicalBlockPool(16, 16)
    cache = v2.PrefixCache(pool)
    request = v2.SequenceState(1, pool)
    request.append_tokens(40)
    prompt = list(range(40))
    cache.publish_computed_block(request, 0, prompt[:16])
    cache.publish_computed_block(request, 1, prompt[:32])
    shared = v2.SequenceState(2, pool)
    prompt[32] = 999
    assert cache.attach_cached_prefix(shared, prompt) == 32
    assert shared.physical_block_id(0) == request.physical_block_id(0)
    assert pool.ref_count(request.block_table().handle(0)) == 2
    with pytest.raises(ValueError):
        cache.publish_computed_block(request, 0, prompt[:16])


def test_prefix_hash_is_fnv1a_over_le_bytes(v2):
    # 64-bit FNV-1a of the 4 little-endian bytes of each token (reference
    # src/block_manager.cpp:214-226), recomputed independently here.
    def fnv(tokens):
        h = 0xcbf29ce484222325
        for t in tokens:
            for byte in (t & 0xffffffff).to_bytes(4, "little"):
                h = ((h ^ byte) * 0x100000001b3) & (2**64 - 1)
        return h

    for tokens in ([], [0], [1, 2, 3], [-1, 2**31 - 1, -(2**31)], list(range(100))):
        assert v2.prefix_hash(tokens) == fnv(tokens)
