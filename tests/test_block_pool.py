"""BlockPool and the block chain hash, host bookkeeping (no GPU needed).

Each test ports one test of the reference's crates/llm-kv-cache/tests/paged_blocks.rs
(named in its docstring) against a bookkeeping-only pool
(BlockPool::new(block_count, capacity, vector_len)); the device payload side
(rows, copy-on-write copies, decode through session tables) is in
test_gpu_block_pool.py.  The chain hash is pinned by the FIPS 180-4 SHA-256
vectors and by an independent restatement over hashlib (oracle.chain_hash).
"""
import hashlib
import threading

import pytest

import llm_hip
import oracle
from llm_hip import BlockPool, LlhError, cache_block_chain_hash

ROOT = bytes(32)


# ---------------------------------------------------------------------------
# SHA-256 and the chain hash


@pytest.mark.parametrize("msg,digest", [
    # FIPS 180-4 example messages (NIST CSRC "SHA256.pdf" examples) and the empty string
    (b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
    (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
    (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
])
def test_sha256_fips_vectors(msg, digest):
    assert llm_hip.sha256(msg).hex() == digest


def test_sha256_matches_hashlib_across_block_boundaries():
    for n in list(range(0, 130)) + [1000, 4096, 1_000_000]:
        data = bytes((i * 131 + 7) & 0xFF for i in range(n))
        assert llm_hip.sha256(data) == hashlib.sha256(data).digest(), n


def test_chain_hash_equals_restated_layout():
    cases = [("model-a", "cache-context-a", ROOT, [11, 12, 13]), ("", "", ROOT, []),
             ("Qwen/Qwen3-0.6B", "ctx", bytes(range(32)), list(range(16))),
             ("m" * 300, "c" * 70, bytes([255]) * 32, [0xFFFFFFFF, 0, 1 << 31])]
    for m, c, prev, toks in cases:
        assert cache_block_chain_hash(m, c, prev, toks) == oracle.chain_hash(m, c, prev, toks)


def test_chain_hash_depends_on_full_prefix_identity():
    """paged_blocks.rs: cache_block_chain_hash_depends_on_full_prefix_identity."""
    first = cache_block_chain_hash("model-a", "cache-context-a", ROOT, [11, 12, 13])
    assert first == cache_block_chain_hash("model-a", "cache-context-a", ROOT, [11, 12, 13])
    assert first != cache_block_chain_hash("model-b", "cache-context-a", ROOT, [11, 12, 13])
    assert first != cache_block_chain_hash("model-a", "cache-context-b", ROOT, [11, 12, 13])
    assert first != cache_block_chain_hash("model-a", "cache-context-a", bytes([1]) * 32, [11, 12, 13])
    assert first != cache_block_chain_hash("model-a", "cache-context-a", ROOT, [11, 12, 99])
    second = cache_block_chain_hash("model-a", "cache-context-a", first, [21, 22])
    changed_parent = cache_block_chain_hash("model-a", "cache-context-a", ROOT, [41, 42])
    assert second != cache_block_chain_hash("model-a", "cache-context-a", changed_parent, [21, 22])


def test_chain_hash_length_prefixes_separate_fields():
    """The u64 length prefixes keep ("ab", "c") and ("a", "bc") apart."""
    assert cache_block_chain_hash("ab", "c", ROOT, [1]) != cache_block_chain_hash("a", "bc", ROOT, [1])


# ---------------------------------------------------------------------------
# BlockPool


def test_block_ids_are_valid_and_unknown_ids_are_absent():
    """paged_blocks.rs: block_id_exposes_invalid_sentinel_without_accepting_it_as_valid."""
    pool = BlockPool.new(2, 4, 3)
    a = pool.allocate()
    assert a and a != 0
    assert pool.block(0) is None
    s = pool.create_session()
    with pytest.raises(LlhError) as e:
        pool.append_block_to_session(s, 0)  # BlockId::INVALID cannot enter a table
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE


def test_shape_errors():
    for shape in [(0, 4, 3), (2, 0, 3), (2, 4, 0)]:
        with pytest.raises(LlhError) as e:
            BlockPool.new(*shape)
        assert e.value.status == llm_hip.ERR_INVALID_SHAPE


def test_allocates_deallocates_and_reuses_free_blocks():
    """paged_blocks.rs: block_pool_allocates_deallocates_and_reuses_free_blocks."""
    pool = BlockPool.new(2, 4, 3)
    assert (pool.total_blocks(), pool.free_blocks(), pool.allocated_blocks()) == (2, 2, 0)
    first, second = pool.allocate(), pool.allocate()
    assert first != second
    assert pool.free_blocks() == 0 and pool.allocated_blocks() == 2
    assert pool.allocate() is None
    assert pool.block(first).ref_count == 1
    pool.commit_tokens(first, 1)  # first_block.append(...) bookkeeping
    assert pool.block(first).token_count == 1
    assert pool.deallocate(first)
    assert pool.free_blocks() == 1 and pool.allocated_blocks() == 1
    assert pool.block(first).token_count == 0 and pool.block(first).ref_count == 0
    reused = pool.allocate()
    assert reused == first
    assert pool.block(reused).token_count == 0 and pool.block(reused).ref_count == 1


def test_release_and_retain_of_free_blocks_fail():
    pool = BlockPool.new(1, 2, 2)
    b = pool.allocate()
    assert pool.release(b)
    assert not pool.release(b)
    assert not pool.retain(b)
    assert pool.touch(b) is None


def test_concurrent_allocation_and_release():
    """paged_blocks.rs: cloned_block_pool_coordinates_concurrent_allocation_and_release."""
    workers, iterations = 8, 64
    pool = BlockPool.new(workers, 2, 2)
    active, lock, errors = set(), threading.Lock(), []
    start = threading.Barrier(workers)

    def work():
        start.wait()
        for _ in range(iterations):
            b = None
            while b is None:
                b = pool.allocate()
            with lock:
                if b in active:
                    errors.append(b)
                active.add(b)
            with lock:
                active.discard(b)
            if not pool.deallocate(b):
                errors.append(-b)

    ts = [threading.Thread(target=work) for _ in range(workers)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    assert pool.allocated_blocks() == 0 and pool.free_blocks() == workers


def test_concurrent_session_allocation_and_release():
    """paged_blocks.rs: cloned_block_pool_coordinates_concurrent_session_allocation_and_release."""
    workers, per_session, iterations = 8, 4, 32
    pool = BlockPool.new(workers * per_session, 2, 2)
    active, lock, errors = set(), threading.Lock(), []
    start = threading.Barrier(workers)

    def work():
        start.wait()
        for _ in range(iterations):
            s = pool.create_session()
            mine = []
            for i in range(per_session):
                b = None
                while b is None:
                    b = pool.allocate_for_session(s)
                if pool.read_session_block(s, i) != b:
                    errors.append(("index", s, i))
                with lock:
                    if b in active:
                        errors.append(("dup", b))
                    active.add(b)
                mine.append(b)
            if pool.session(s).owned_block_count != per_session:
                errors.append(("owned", s))
            with lock:
                for b in mine:
                    active.discard(b)
            if not pool.release_session(s) or pool.session(s) is not None:
                errors.append(("release", s))

    ts = [threading.Thread(target=work) for _ in range(workers)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors and not active
    assert pool.session_count() == 0 and pool.allocated_blocks() == 0
    assert pool.free_blocks() == workers * per_session


def test_lru_access_order_for_allocated_blocks():
    """paged_blocks.rs: block_pool_maintains_lru_access_order_for_allocated_blocks."""
    pool = BlockPool.new(3, 2, 2)
    first, second, third = pool.allocate(), pool.allocate(), pool.allocate()
    assert pool.lru_block() == first
    assert pool.touch(first)
    assert pool.lru_block() == second
    assert pool.touch(second)
    assert pool.lru_block() == third
    assert pool.deallocate(third)
    assert pool.lru_block() == first
    assert pool.block(third).last_access == 0


def test_sessions_create_and_release_return_owned_blocks():
    """paged_blocks.rs: block_pool_creates_sessions_and_release_returns_owned_blocks."""
    pool = BlockPool.new(3, 2, 2)
    s1, s2 = pool.create_session(), pool.create_session()
    assert s1 != s2 and pool.session_count() == 2
    assert pool.session(s1).session_id == s1
    assert pool.session(s1).created_at < pool.session(s2).created_at
    b1, b2 = pool.allocate_for_session(s1), pool.allocate_for_session(s1)
    b3 = pool.allocate_for_session(s2)
    assert len({b1, b2, b3}) == 3
    assert pool.free_blocks() == 0 and pool.allocated_blocks() == 3
    assert pool.session(s1).block_count == 2 and pool.session(s1).owned_block_count == 2
    assert pool.release_session(s1)
    assert pool.session(s1) is None and pool.session_count() == 1
    assert pool.free_blocks() == 2 and pool.allocated_blocks() == 1
    assert pool.block(b1).ref_count == 0 and pool.block(b2).ref_count == 0 and pool.block(b3).ref_count == 1
    assert pool.allocate_for_session(s2) in (b1, b2)
    assert not pool.release_session(s1)


def _prefix(pool, owner, hashes):
    blocks = []
    for h in hashes:
        b = pool.allocate_for_session(owner)
        pool.set_content_hash(b, h)
        blocks.append(b)
    return blocks


def test_prefix_lookup_and_attach_share_registered_blocks():
    """paged_blocks.rs: block_pool_prefix_lookup_and_attach_share_registered_blocks."""
    pool = BlockPool.new(3, 2, 2)
    owner, reader = pool.create_session(), pool.create_session()
    h1 = cache_block_chain_hash("model-a", "cache-context-a", ROOT, [1, 2])
    h2 = cache_block_chain_hash("model-a", "cache-context-a", h1, [3, 4])
    first, second = _prefix(pool, owner, [h1, h2])
    pool.register_prefix(h2, [first, second])
    assert pool.lookup_prefix(h2) == [first, second]
    assert pool.attach_prefix_to_session(reader, h2) == [first, second]
    assert pool.read_session_block(reader, 0) == first and pool.read_session_block(reader, 1) == second
    assert pool.block(first).ref_count == 2 and pool.block(second).ref_count == 2


def test_register_prefix_requires_matching_terminal_hash():
    pool = BlockPool.new(3, 2, 2)
    owner = pool.create_session()
    h1 = cache_block_chain_hash("m", "c", ROOT, [1, 2])
    h2 = cache_block_chain_hash("m", "c", h1, [3, 4])
    first, second = _prefix(pool, owner, [h1, h2])
    pool.register_prefix(h1, [first, second])  # terminal hash is h2, not h1
    assert pool.lookup_prefix(h1) is None
    pool.register_prefix(h2, [first, second])
    assert pool.lookup_prefix(h2) == [first, second]
    pool.set_content_hash(second, None)  # hashes cleared: re-registering removes the entry
    pool.register_prefix(h2, [first, second])
    assert pool.lookup_prefix(h2) is None


def test_prefix_attach_misses_when_intermediate_block_is_reused():
    """paged_blocks.rs: block_pool_prefix_attach_misses_when_intermediate_block_is_reused_with_different_hash."""
    pool = BlockPool.new(3, 2, 2)
    owner = pool.create_session()
    h1 = cache_block_chain_hash("model-a", "cache-context-a", ROOT, [1, 2])
    h2 = cache_block_chain_hash("model-a", "cache-context-a", h1, [3, 4])
    reused_hash = cache_block_chain_hash("model-a", "cache-context-a", ROOT, [99, 100])
    first, second = _prefix(pool, owner, [h1, h2])
    pool.register_prefix(h2, [first, second])
    assert pool.release(first)
    recycler = pool.create_session()
    reused = pool.allocate_for_session(recycler)
    assert reused == first
    pool.set_content_hash(reused, reused_hash)
    rc1, rc2 = pool.block(first).ref_count, pool.block(second).ref_count
    reader = pool.create_session()
    assert pool.lookup_prefix(h2) is None
    assert pool.attach_prefix_to_session(reader, h2) is None
    assert pool.block(first).ref_count == rc1 and pool.block(second).ref_count == rc2
    assert pool.session(reader).block_count == 0


def test_releasing_session_decrements_shared_refcounts_once():
    """paged_blocks.rs: releasing_session_decrements_owned_shared_block_refcounts_once."""
    pool = BlockPool.new(1, 2, 2)
    owner, reader = pool.create_session(), pool.create_session()
    shared = pool.allocate_for_session(owner)
    pool.append_block_to_session(reader, shared)
    pool.append_block_to_session(reader, shared)
    assert pool.block(shared).ref_count == 2
    assert pool.session(reader).block_count == 2 and pool.session(reader).owned_block_count == 1
    assert pool.release_session(owner)
    assert pool.block(shared).ref_count == 1 and pool.free_blocks() == 0
    assert pool.read_session_block(reader, 0) == shared and pool.read_session_block(reader, 1) == shared
    assert pool.release_session(reader)
    assert pool.block(shared).ref_count == 0 and pool.free_blocks() == 1


def test_shared_block_is_not_directly_mutable_without_cow():
    """paged_blocks.rs: shared_session_block_is_not_directly_mutable_without_cow."""
    pool = BlockPool.new(2, 2, 2)
    owner, writer = pool.create_session(), pool.create_session()
    shared = pool.allocate_for_session(owner)
    pool.append_block_to_session(writer, shared)
    assert pool.block(shared).ref_count == 2
    for mutate in (lambda: pool.set_content_hash(shared, bytes(32)), lambda: pool.commit_tokens(shared, 1)):
        with pytest.raises(LlhError) as e:
            mutate()
        assert e.value.status == llm_hip.ERR_INVALID_SHAPE


def test_copy_on_write_clones_shared_block_on_first_write():
    """paged_blocks.rs: copy_on_write_session_block_clones_shared_prefix_on_first_write (bookkeeping)."""
    pool = BlockPool.new(3, 2, 2)
    reader, writer = pool.create_session(), pool.create_session()
    shared = pool.allocate_for_session(reader)
    pool.commit_tokens(shared, 1)
    pool.append_block_to_session(writer, shared)
    wb = pool.copy_on_write_session_block(writer, 0)
    assert wb != shared
    assert pool.read_session_block(reader, 0) == shared and pool.read_session_block(writer, 0) == wb
    assert pool.block(shared).ref_count == 1 and pool.block(wb).ref_count == 1
    assert pool.block(wb).token_count == 1  # contents copied
    pool.commit_tokens(wb, 1)
    assert pool.block(shared).token_count == 1 and pool.block(wb).token_count == 2
    # an exclusive block needs no copy
    assert pool.copy_on_write_session_block(writer, 0) == wb


def test_releasing_last_session_after_cow_returns_all_blocks():
    """paged_blocks.rs: releasing_last_session_after_cow_returns_all_blocks_to_free_list."""
    pool = BlockPool.new(2, 2, 2)
    reader, writer = pool.create_session(), pool.create_session()
    shared = pool.allocate_for_session(reader)
    pool.append_block_to_session(writer, shared)
    wb = pool.copy_on_write_session_block(writer, 0)
    assert pool.free_blocks() == 0
    assert pool.release_session(reader)
    assert pool.block(shared).ref_count == 0 and pool.block(wb).ref_count == 1 and pool.free_blocks() == 1
    assert pool.release_session(writer)
    assert pool.block(wb).ref_count == 0 and pool.free_blocks() == 2


def test_cow_evicts_other_sessions_before_copying():
    pool = BlockPool.new(1, 2, 2)
    a, b = pool.create_session(), pool.create_session()
    blk = pool.allocate_for_session(a)
    pool.append_block_to_session(b, blk)
    # no free block: evicting the LRU other session drops the share, so no copy is needed
    assert pool.copy_on_write_session_block(b, 0) == blk
    assert pool.session(a) is None and pool.block(blk).ref_count == 1
    with pytest.raises(LlhError) as e:
        pool.copy_on_write_session_block(b, 5)
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE


def test_cow_without_a_free_block_reports_capacity():
    pool = BlockPool.new(1, 2, 2)
    s = pool.create_session()
    blk = pool.allocate_for_session(s)
    assert pool.retain(blk)  # a holder outside any session: nothing to evict
    with pytest.raises(LlhError) as e:
        pool.copy_on_write_session_block(s, 0)
    assert e.value.status == llm_hip.ERR_CAPACITY
    assert pool.block(blk).ref_count == 2 and pool.read_session_block(s, 0) == blk


def test_full_pool_evicts_least_recently_used_session():
    """paged_blocks.rs: full_pool_evicts_least_recently_used_session_before_allocating."""
    pool = BlockPool.new(2, 2, 2)
    cold, hot = pool.create_session(), pool.create_session()
    cold_block = pool.allocate_for_session(cold)
    hot_block = pool.allocate_for_session(hot)
    assert pool.lru_session() == cold
    assert pool.read_session_block(hot, 0) == hot_block
    assert pool.lru_session() == cold
    newcomer = pool.create_session()
    assert pool.allocate_for_session(newcomer) == cold_block
    assert pool.session(cold) is None and pool.session(hot) is not None and pool.session(newcomer) is not None
    assert pool.block(hot_block).ref_count == 1
    assert pool.total_blocks() == 2 and pool.free_blocks() == 0


def test_multiple_sessions_read_independent_tables():
    """paged_blocks.rs: multiple_sessions_read_independent_block_tables_safely (bookkeeping)."""
    pool = BlockPool.new(2, 2, 2)
    first, second = pool.create_session(), pool.create_session()
    b1, b2 = pool.allocate_for_session(first), pool.allocate_for_session(second)
    assert pool.read_session_block(first, 0) == b1 and pool.read_session_block(second, 0) == b2
    assert pool.release_session(first)
    assert pool.read_session_block(second, 0) == b2 and pool.block(b2).ref_count == 1
    assert pool.read_session_block(second, 1) is None
    assert pool.read_session_block(first, 0) is None


def test_metrics_track_sharing_cow_eviction_and_utilization():
    """paged_blocks.rs: block_pool_metrics_track_sharing_cow_eviction_and_utilization."""
    pool = BlockPool.new(3, 2, 2)
    m = pool.metrics_snapshot()
    assert (m.total_blocks, m.resident_blocks, m.active_blocks, m.free_list_blocks) == (3, 0, 0, 3)
    assert m.pool_utilization_pct == 0.0 and m.total_refcount_increments == 0 and m.pool_high_water_blocks == 0
    owner, reader = pool.create_session(), pool.create_session()
    first, second = pool.allocate_for_session(owner), pool.allocate_for_session(owner)
    pool.commit_tokens(first, 1)
    pool.append_block_to_session(reader, first)
    m = pool.metrics_snapshot()
    assert (m.resident_blocks, m.active_blocks, m.shared_blocks, m.refcount_total) == (2, 3, 1, 3)
    assert (m.max_refcount_seen, m.total_refcount_increments, m.cow_bytes_saved) == (2, 1, 32)
    assert (m.free_list_blocks, m.pool_high_water_blocks) == (1, 2)
    assert abs(m.avg_refcount - 1.5) < 1e-15
    assert abs(m.pool_utilization_pct - 66.66666666666666) < 1e-12
    rb = pool.copy_on_write_session_block(reader, 0)
    assert rb != first
    m = pool.metrics_snapshot()
    assert (m.resident_blocks, m.active_blocks, m.shared_blocks, m.total_cow_clones) == (3, 3, 0, 1)
    assert (m.cow_bytes_saved, m.pool_high_water_blocks, m.free_list_blocks) == (32, 3, 0)
    newcomer = pool.create_session()
    assert pool.allocate_for_session(newcomer) in (first, second)
    assert pool.session(owner) is None
    m = pool.metrics_snapshot()
    assert (m.sessions, m.resident_blocks, m.active_blocks) == (2, 2, 2)
    assert (m.blocks_evicted_lru, m.sessions_evicted_lru, m.eviction_high_water_mark) == (2, 1, 3)
    assert m.pool_high_water_blocks == 3


def test_metrics_reset_when_pool_is_recreated():
    """paged_blocks.rs: block_pool_metrics_reset_when_pool_is_recreated."""
    pool = BlockPool.new(1, 2, 2)
    s = pool.create_session()
    pool.allocate_for_session(s)
    m = pool.metrics_snapshot()
    assert m.resident_blocks == 1 and m.pool_high_water_blocks == 1
    m = BlockPool.new(1, 2, 2).metrics_snapshot()
    assert (m.total_blocks, m.resident_blocks, m.active_blocks, m.total_refcount_increments) == (1, 0, 0, 0)
    assert (m.total_cow_clones, m.blocks_evicted_lru, m.pool_high_water_blocks) == (0, 0, 0)


def test_admin_view_of_session_tables_and_refcounts():
    """paged_blocks.rs: block_pool_admin_snapshot_includes_session_block_tables_and_refcounts."""
    pool = BlockPool.new(2, 2, 2)
    owner, reader = pool.create_session(), pool.create_session()
    shared = pool.allocate_for_session(owner)
    pool.append_block_to_session(reader, shared)
    m = pool.metrics_snapshot()
    assert m.total_blocks == 2 and m.shared_blocks == 1 and m.sessions == 2
    for s in (owner, reader):
        ids, idx = pool.session_blocks(s)
        assert ids == [shared] and pool.block(shared).ref_count == 2
        assert idx.tolist() == [pool.block(shared).pool_index]
