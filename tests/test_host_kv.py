"""Host-side bookkeeping: the reference's own unit tests, ported one for one
(kv_pool.rs:104-162, radix_cache.rs:305-425), then the block manager that
feeds the device pool (refcounts, decode growth, copy-on-write, compaction).
CPU only."""
from __future__ import annotations

import time

import numpy as np
import pytest

from mitten_amd.host import BlockManager, DoubleFree, KvCachePool, OutOfBlocks, PageTable, RadixCache

# ---------------------------------------------- kv_pool.rs:104-162 (ported) ----


def test_allocate_and_free():
    pool = KvCachePool(16, 16)
    p1 = pool.allocate(1)
    assert pool.free_pages() == 15
    pool.free(p1)
    assert pool.free_pages() == 16


def test_allocate_exhaustion():
    pool = KvCachePool(2, 16)
    assert pool.allocate(1) is not None
    assert pool.allocate(1) is not None
    assert pool.allocate(1) is None
    assert pool.free_pages() == 0


def test_required_bytes():
    assert KvCachePool.required_bytes(1, 16, 1, 1, 1, 1) == 32
    assert KvCachePool.required_bytes(512, 16, 28, 4, 128, 2) == 2 * 512 * 16 * 28 * 4 * 128 * 2


def test_double_free_panics():
    pool = KvCachePool(4, 16)
    p = pool.allocate(1)
    pool.free(p)
    with pytest.raises(DoubleFree):
        pool.free(p)


def test_page_table_roundtrip():
    pt = PageTable()
    pt.insert(7, 0, 7)
    assert pt.lookup(7, 0) == 7
    assert pt.remove_request(7) == [7]
    assert pt.lookup(7, 0) is None


def test_allocation_order_and_lifo_reuse():
    """new() reverses 0..n so pages come out 0,1,2,... (kv_pool.rs:19-20);
    a freed page is the next one handed out (stack)."""
    pool = KvCachePool(5, 16)
    assert [pool.allocate(1) for _ in range(3)] == [0, 1, 2]
    pool.free(1)
    pool.free(0)
    assert pool.allocate(2) == 0 and pool.allocate(2) == 1 and pool.allocate(2) == 3


# ------------------------------------------ radix_cache.rs:305-425 (ported) ----


def test_empty_match():
    cache = RadixCache(4, 16)
    length, pages, nodes = cache.match_prefix([1, 2, 3])
    assert length == 0 and pages == [] and nodes == []


def test_insert_and_match_full():
    cache = RadixCache(4, 16)
    cache.insert_prefix([1, 2, 3, 4], [10])
    length, pages, nodes = cache.match_prefix([1, 2, 3, 4, 5])
    assert length == 4 and pages == [10] and len(nodes) == 1


def test_edge_split():
    cache = RadixCache(2, 16)
    cache.insert_prefix([1, 2, 3, 4], [10, 11])
    cache.insert_prefix([1, 2, 5, 6], [10, 12])
    l1, p1, _ = cache.match_prefix([1, 2, 3, 4])
    assert l1 == 4 and p1 == [10, 11]
    l2, p2, _ = cache.match_prefix([1, 2, 5, 6])
    assert l2 == 4 and p2 == [10, 12]


def test_lru_eviction():
    cache = RadixCache(2, 2)
    cache.insert_prefix([1, 2], [10])
    cache.insert_prefix([3, 4], [11])
    assert cache.total_cached_pages() == 2
    cache.insert_prefix([5, 6], [12])  # evicts [1, 2]
    assert cache.total_cached_pages() == 2
    length, _, _ = cache.match_prefix([1, 2])
    assert length == 0
    assert cache.take_evicted() == [10]  # returned, not leaked (reference drops it)


def test_lock_prevents_eviction():
    cache = RadixCache(2, 1)
    cache.insert_prefix([1, 2], [10])
    _, _, nodes = cache.match_prefix([1, 2])
    cache.insert_prefix([3, 4], [11])
    assert cache.total_cached_pages() == 2  # overflowed: nothing was evictable
    cache.unlock_nodes(nodes)
    freed = cache.evict_pages(1)
    assert len(freed) == 1


def test_insert_and_match_partial_edge():
    cache = RadixCache(4, 16)
    cache.insert_prefix([1, 2, 3, 4], [10])
    cache.insert_prefix([1, 2, 5, 6], [11])
    length, pages, _ = cache.match_prefix([1, 2, 3, 4])
    assert len(pages) == length // 4
    length2, pages2, _ = cache.match_prefix([1, 2, 5, 6])
    assert len(pages2) == length2 // 4


def test_promote_request():
    cache = RadixCache(8, 16)
    cache.promote_request(list(range(1, 9)), 8, [42])
    length, pages, _ = cache.match_prefix(list(range(1, 9)))
    assert length == 8 and pages == [42]


def test_page_alignment():
    cache = RadixCache(4, 16)
    cache.insert_prefix([1, 2, 3, 4, 5, 6], [10])
    length, pages, _ = cache.match_prefix([1, 2, 3, 4, 5, 6])
    assert length == 4 and pages == [10]


# ------------------------------------------------- radix: further semantics ----


def test_split_creates_intermediate_node_and_keeps_pages():
    cache = RadixCache(2, 16)
    cache.insert_prefix([1, 2, 3, 4, 5, 6], [10, 11, 12])
    assert cache.num_nodes() == 2  # root + leaf
    cache.insert_prefix([1, 2, 3, 4, 7, 8], [10, 11, 13])
    assert cache.num_nodes() == 4  # root, [1..4], [5,6], [7,8]
    assert cache.total_cached_pages() == 4
    assert cache.match_prefix([1, 2, 3, 4, 5, 6])[1] == [10, 11, 12]
    assert cache.match_prefix([1, 2, 3, 4, 7, 8])[1] == [10, 11, 13]


def test_eviction_order_follows_the_lazy_heap():
    """The LRU heap holds stale entries (radix_cache.rs:40,160,233-234): an entry
    is skipped only if its node is gone or not evictable (:250-255). So a leaf
    touched after insertion is still evicted at its insertion stamp, first."""
    cache = RadixCache(2, 8)
    for i, t in enumerate(([1, 2], [3, 4], [5, 6])):
        cache.insert_prefix(t, [10 + i])
    _, _, n = cache.match_prefix([1, 2])
    cache.unlock_nodes(n)
    assert cache.evict_pages(1) == [10]
    assert cache.evict_pages(1) == [11]
    assert cache.evict_pages(1) == [12]
    assert cache.evict_pages(1) == []


def test_locked_leaf_is_skipped_until_unlocked():
    cache = RadixCache(2, 8)
    for i, t in enumerate(([1, 2], [3, 4])):
        cache.insert_prefix(t, [10 + i])
    _, _, n = cache.match_prefix([1, 2])
    assert cache.evict_pages(1) == [11]
    assert cache.evict_pages(1) == []  # [1,2] locked; its heap entry was consumed
    cache.unlock_nodes(n)  # re-queued on unlock
    assert cache.evict_pages(1) == [10]


def test_parent_becomes_evictable_after_children_go():
    cache = RadixCache(2, 8)
    cache.insert_prefix([1, 2, 3, 4], [10, 11])
    cache.insert_prefix([1, 2, 5, 6], [10, 12])
    freed = cache.evict_pages(3)
    assert sorted(freed) == [10, 11, 12]
    assert cache.total_cached_pages() == 0 and cache.num_nodes() == 1


# ---------------------------------------------------------- block manager ----


def _tokens(seed, n):
    return np.random.default_rng(seed).integers(0, 50_000, n).astype(np.uint32)


def test_block_manager_refuses_pools_whose_slots_overflow_int32():
    """Slots are block * page_size + offset in int32 (the device pool's slot
    type): 2^27 blocks of 16 tokens, or 2^20 of 2,048, would wrap them."""
    from mitten_amd.host import INVALID_ARGUMENT, HostError

    BlockManager(2**20 - 1, 2048, max_cached_pages=0).close()
    for n, ps in ((2**27, 16), (2**20, 2048)):
        with pytest.raises(HostError) as ei:
            BlockManager(n, ps)
        assert ei.value.status == INVALID_ARGUMENT and "int32" in str(ei.value)


def test_admit_allocates_ceil_pages_and_decode_grows():
    bm = BlockManager(64, 16)
    assert bm.admit(1, _tokens(0, 40)) == 0
    assert len(bm.table(1)) == 3
    slots, cow = bm.append(1, 40)  # the prompt's K/V
    assert cow == [] and bm.seq_len(1) == 40
    t = bm.table(1)
    assert list(slots) == [t[p // 16] * 16 + p % 16 for p in range(40)]
    for step in range(30):  # decode: a block is added whenever pos % 16 == 0
        s, _ = bm.append(1, 1)
        pos = 40 + step
        assert s[0] == bm.table(1)[pos // 16] * 16 + pos % 16
    assert len(bm.table(1)) == (70 + 15) // 16
    bm.check_invariants()


def test_radix_sharing_refcounts_and_no_double_free():
    """A finished request's promoted pages stay in the tree; releasing the
    request must not free them (the reference frees them twice: scheduler.rs:169
    and later eviction)."""
    bm = BlockManager(32, 16)
    toks = _tokens(1, 64)
    bm.admit(1, toks)
    bm.append(1, 64)
    bm.promote(1, toks)
    assert bm.cached_pages() == 4
    assert all(bm.refcount(b) == 2 for b in bm.table(1))
    bm.release(1)
    assert bm.free_blocks() == 28
    bm.check_invariants()
    cached = bm.admit(2, np.concatenate([toks, _tokens(2, 20)]))
    assert cached == 64
    assert all(bm.refcount(b) == 2 for b in bm.table(2)[:4])
    bm.append(2, 20)
    bm.check_invariants()
    bm.release(2)
    assert bm.evict(100) == 4
    assert bm.free_blocks() == 32
    bm.check_invariants()


def test_fork_then_copy_on_write_of_shared_partial_block():
    bm = BlockManager(16, 16)
    bm.admit(1, _tokens(3, 20))
    bm.append(1, 20)  # blocks: [full, partial(4 tokens)]
    bm.fork(1, 2)
    t1, t2 = bm.table(1), bm.table(2)
    assert list(t1) == list(t2) and all(bm.refcount(b) == 2 for b in t1)
    slots, cow = bm.append(2, 1)  # writes into the shared partial block -> copy first
    assert len(cow) == 1 and cow[0][0] == t1[1]
    assert bm.table(2)[1] == cow[0][1] != t1[1]
    assert slots[0] == cow[0][1] * 16 + 4
    slots1, cow1 = bm.append(1, 1)  # last holder writes in place
    assert cow1 == [] and slots1[0] == t1[1] * 16 + 4
    bm.check_invariants()


def test_fork_before_the_prompt_is_written_gives_private_blocks():
    """Admission reserves ceil(n/16) blocks; a fork made before any of them is
    written shares them all. Each sequence's append must then write only
    blocks it alone holds, and nothing needs copying (no rows exist yet)."""
    bm = BlockManager(16, 16)
    bm.admit(1, _tokens(21, 40))
    bm.fork(1, 2)
    assert all(bm.refcount(b) == 2 for b in bm.table(1))
    s1, c1 = bm.append(1, 40)
    s2, c2 = bm.append(2, 40)
    assert c1 == [] and c2 == []
    assert set(s1.tolist()).isdisjoint(s2.tolist())
    for s in (s1, s2):
        assert all(bm.refcount(int(x) // 16) == 1 for x in s)
    assert set(bm.table(1).tolist()).isdisjoint(bm.table(2).tolist())
    bm.check_invariants()


def test_fork_during_prefill_copies_only_the_partial_block():
    """Fork after 20 of 40 prompt tokens: block 0 is full (shared, never
    written again), block 1 holds 4 rows (copy on write), block 2 holds none
    (a fresh private block, no copy)."""
    bm = BlockManager(16, 16)
    bm.admit(1, _tokens(22, 40))
    bm.append(1, 20)
    t = bm.table(1).copy()
    bm.fork(1, 2)
    s2, c2 = bm.append(2, 20)
    assert c2 == [(int(t[1]), int(bm.table(2)[1]))]
    t2 = bm.table(2)
    assert t2[0] == t[0] and t2[1] != t[1] and t2[2] != t[2]
    s1, c1 = bm.append(1, 20)  # now the last holder of blocks 1 and 2: in place
    assert c1 == [] and list(bm.table(1)) == list(t)
    assert set(s1.tolist()).isdisjoint(s2.tolist())
    assert bm.refcount(int(t[0])) == 2
    bm.check_invariants()


def test_compaction_without_outputs_is_refused_and_changes_nothing():
    import ctypes

    from mitten_amd import host as hm

    bm = BlockManager(40, 16)
    for s in range(6):
        bm.admit(s, _tokens(30 + s, 40))
        bm.append(s, 40)
    bm.release(1)
    tables = {s: bm.table(s).copy() for s in (0, 2, 3, 4, 5)}
    n = ctypes.c_int64()
    st = hm._lib_h().mkvh_bm_plan_compaction(bm._h, None, None, 40, ctypes.byref(n))
    assert st != 0 and b"out_src" in hm._lib_h().mkvh_last_error()
    for s, t in tables.items():
        assert list(bm.table(s)) == list(t)
    bm.check_invariants()


def test_compaction_moves_tail_blocks_into_holes():
    bm = BlockManager(40, 16)
    for s in range(8):
        bm.admit(s, _tokens(10 + s, 50))
        bm.append(s, 50)
    for s in (1, 4, 6):
        bm.release(s)
    live = bm.live_blocks()
    before = {s: bm.table(s).copy() for s in (0, 2, 3, 5, 7)}
    src, dst = bm.plan_compaction()
    assert len(src) == len(dst) and set(src).isdisjoint(dst)
    assert all(d < live for d in dst) and all(s >= live for s in src)
    moved = dict(zip(src.tolist(), dst.tolist()))
    for s, t in before.items():
        assert list(bm.table(s)) == [moved.get(b, b) for b in t]
        assert max(bm.table(s)) < live
    bm.check_invariants()
    bm.admit(99, _tokens(99, 16))
    assert bm.table(99)[0] == live  # free ids are now exactly [live, N)


def test_admission_exhaustion_is_reported_and_changes_nothing():
    bm = BlockManager(4, 16)
    bm.admit(1, _tokens(4, 48))
    with pytest.raises(OutOfBlocks):
        bm.admit(2, _tokens(5, 32))
    assert bm.free_blocks() == 1
    bm.check_invariants()


def test_batch_metadata_matches_tables():
    bm = BlockManager(64, 16)
    for s, n in ((5, 10), (6, 33), (7, 16)):
        bm.admit(s, _tokens(s, n))
        bm.append(s, n)
    indptr, ids, ctx = bm.batch([6, 5, 7])
    assert list(ctx) == [33, 10, 16]
    assert list(ids[indptr[0]:indptr[1]]) == list(bm.table(6))
    assert list(ids[indptr[2]:indptr[3]]) == list(bm.table(7))


def test_scheduler_overhead_bound():
    """scheduler_bench.rs:46-79 analogue: 1000 decode iterations over 32
    sequences (append + batch metadata) within 1000 ms."""
    bm = BlockManager(4096, 16)
    seqs = list(range(32))
    for s in seqs:
        bm.admit(s, _tokens(100 + s, 16))
        bm.append(s, 16)
    t0 = time.perf_counter()
    for _ in range(1000):
        for s in seqs:
            bm.append(s, 1)
        bm.batch(seqs)
    assert time.perf_counter() - t0 < 1.0
    bm.check_invariants()


def test_random_lifecycle_keeps_invariants():
    rng = np.random.default_rng(7)
    bm = BlockManager(256, 16, max_cached_pages=64)
    live, next_id, prompts = set(), 0, {}
    shared = _tokens(999, 64)
    for it in range(400):
        op = rng.integers(0, 5)
        if op == 0 or not live:
            n = int(rng.integers(1, 80))
            toks = np.concatenate([shared[: int(rng.integers(0, 65))], _tokens(it, n)])
            try:
                cached = bm.admit(next_id, toks)
            except OutOfBlocks:
                continue
            bm.append(next_id, len(toks) - cached)
            prompts[next_id] = toks
            live.add(next_id)
            next_id += 1
        elif op == 1:
            s = int(rng.choice(sorted(live)))
            if rng.integers(0, 3) == 0:  # fork it, then let either side write
                c = next_id
                bm.fork(s, c)
                prompts[c] = prompts[s]
                live.add(c)
                next_id += 1
                s = int(rng.choice([s, c]))
            try:
                slots, _ = bm.append(s, int(rng.integers(1, 20)))
            except OutOfBlocks:
                pass
            else:  # every block written is held by the writer alone
                assert all(bm.refcount(int(x) // 16) == 1 for x in slots)
        elif op == 2:
            s = int(rng.choice(sorted(live)))
            bm.promote(s, prompts[s])
        elif op == 3:
            s = int(rng.choice(sorted(live)))
            bm.release(s)
            live.discard(s)
        else:
            bm.evict(int(rng.integers(1, 8)))
        bm.check_invariants()
    bm.plan_compaction()
    bm.check_invariants()


def test_split_shared_prefix_tables():
    from mitten_amd.host import split_shared_prefix

    # three tables sharing blocks 7, 8, 9; the third diverges at its 4th block
    ip = np.array([0, 5, 10, 14], np.int32)
    ids = np.array([7, 8, 9, 1, 2, 7, 8, 9, 1, 3, 7, 8, 9, 4], np.int32)
    ctx = np.array([70, 80, 60], np.int32)
    pre, sp, si, sl = split_shared_prefix(ip, ids, ctx)
    assert pre.tolist() == [7, 8, 9]
    assert sp.tolist() == [0, 2, 4, 5] and si.tolist() == [1, 2, 1, 3, 4] and sl.tolist() == [22, 32, 12]
    # a sequence whose last token sits in a shared block caps the prefix
    pre, sp, si, sl = split_shared_prefix(ip, ids, np.array([70, 80, 48], np.int32))
    assert pre.tolist() == [7, 8] and sl.tolist() == [38, 48, 16]
    # nothing shared
    pre, sp, si, sl = split_shared_prefix(np.array([0, 1, 2], np.int32), np.array([5, 6], np.int32),
                                          np.array([3, 4], np.int32))
    assert pre.size == 0 and si.tolist() == [5, 6] and sl.tolist() == [3, 4]


def test_block_manager_shared_prefix_after_fork():
    """Forked sequences share the prefix's full pages (refcounted); the
    split puts exactly those in the prefix and every suffix starts with the
    sequence's own pages."""
    bm = BlockManager(64)
    assert bm.admit(0, np.arange(100, dtype=np.uint32)) == 0
    bm.append(0, 100)  # 6 full pages + 4 tokens
    for s in (1, 2):
        bm.fork(0, s)
    for s in (0, 1, 2):
        bm.append(s, 5 + s)  # COW of the partial page for all but its last holder
    pre, sp, si, sl = bm.batch_shared_prefix([0, 1, 2])
    assert pre.tolist() == list(bm.table(0)[:6]) and all(bm.refcount(int(b)) == 3 for b in pre)
    assert sl.tolist() == [100 + 5 - 96, 100 + 6 - 96, 100 + 7 - 96]
    own = [si[sp[b]:sp[b + 1]] for b in range(3)]
    assert len({int(o[0]) for o in own}) == 3  # each sequence's own copy of the partial page


# ------------------------------ PrefillAdder's budget (prefill.rs:21-114) ----


@pytest.mark.parametrize("budget,remaining,chunks,used", [
    # In order, min(remaining, budget - used): the second request gets what is left.
    (100, [30, 200, 5], [30, 70, 0], 100),
    # The loop stops once the budget is used up (prefill.rs:28-30).
    (10, [10, 4], [10, 0], 10),
    # A request with nothing left gets no chunk and uses no budget (:101-104).
    (64, [0, 40, 40], [0, 40, 24], 64),
    # Budget 0: nothing is scheduled.
    (0, [16, 16], [0, 0], 0),
    # The pool-pressure step: 8 prefills with a 512-token chunk left each
    # fill a budget of 4,096; a ninth waits.
    (4096, [512] * 9, [512] * 8 + [0], 4096),
])
def test_prefill_chunk_rule_hand_worked(budget, remaining, chunks, used):
    from mitten_amd.host import schedule_prefill_chunks

    got, u = schedule_prefill_chunks(budget, remaining)
    assert got == chunks and u == used


def test_prefill_chunk_rule_matches_a_loop_restatement():
    """Random cases against a plain restatement of prefill.rs:27-36 + 99-114."""
    from mitten_amd.host import schedule_prefill_chunks

    rng = np.random.default_rng(5)
    for _ in range(200):
        rem = rng.integers(0, 300, rng.integers(0, 12)).tolist()
        budget = int(rng.integers(0, 1200))
        want, used = [0] * len(rem), 0
        for i, r in enumerate(rem):
            if used >= budget:
                break
            c = min(r, budget - used)
            if r > 0 and c > 0:
                want[i] = c
                used += c
        assert schedule_prefill_chunks(budget, rem) == (want, used)


def test_schedule_prefill_in_progress_first_then_admission():
    """Two prefills in progress (prompts 100 and 300 tokens, 40 and 0 written)
    and two waiting prompts. Budget 320: the in-progress ones get 60 and
    min(300, 260) = 260 in order, and no waiting request is admitted, since
    admission needs budget left (prefill.rs:39). Budget 400: 60 and 300, then
    the first waiting request is admitted and gets the 40 tokens left; the
    second is not admitted."""
    bm = BlockManager(256, 16)
    bm.admit(1, _tokens(1, 100))
    bm.append(1, 40)
    bm.admit(2, _tokens(2, 300))
    waiting = [(3, _tokens(3, 200)), (4, _tokens(4, 50))]
    ip, wc, n_adm, cached = bm.schedule_prefill(320, [1, 2], waiting)
    assert ip == [60, 260] and n_adm == 0 and wc == [0, 0] and cached == []
    ip, wc, n_adm, cached = bm.schedule_prefill(400, [1, 2], waiting)
    assert ip == [60, 300] and n_adm == 1 and wc == [40, 0] and cached == [0]
    assert bm.seq_len(3) == 0  # admitted: blocks reserved, nothing written yet
    bm.append(3, 40)
    bm.check_invariants()


def test_schedule_prefill_admission_stops_at_the_first_that_does_not_fit():
    """The reference breaks out of admission at the first request the pool
    cannot hold (prefill.rs:51-54), even when a later, smaller one would fit."""
    bm = BlockManager(10, 16)
    waiting = [(1, _tokens(1, 64)), (2, _tokens(2, 200)), (3, _tokens(3, 16))]
    ip, wc, n_adm, cached = bm.schedule_prefill(10_000, [], waiting)
    assert n_adm == 1 and wc == [64, 0, 0] and ip == []
    assert bm.free_blocks() == 6
    bm.check_invariants()


def test_schedule_prefill_radix_hit_starts_the_chunk_after_the_cached_prefix():
    """A waiting prompt whose first 32 tokens are in the tree is admitted with
    cached length 32 and chunked from there; a prompt cached in full gets no
    chunk (the reference's remaining == 0 case)."""
    bm = BlockManager(64, 16)
    p = _tokens(7, 32)
    bm.admit(1, p)
    bm.append(1, 32)
    bm.promote(1, p)
    bm.release(1)
    longer = np.concatenate([p, _tokens(8, 20)])
    ip, wc, n_adm, cached = bm.schedule_prefill(15, [], [(2, longer), (3, p)])
    assert n_adm == 1 and cached == [32] and wc == [15, 0]
    bm.append(2, 15)  # the step writes the chunk
    ip, wc, n_adm, cached = bm.schedule_prefill(100, [2], [(3, p)])
    assert ip == [5] and n_adm == 1 and cached == [32] and wc == [0]
    bm.check_invariants()


def test_schedule_prefill_refuses_bad_arguments_before_changing_anything():
    from mitten_amd.host import HostError

    bm = BlockManager(32, 16)
    bm.admit(1, _tokens(1, 20))
    free = bm.free_blocks()
    with pytest.raises(HostError):
        bm.schedule_prefill(100, [9], [(2, _tokens(2, 20))])  # unknown in-progress sequence
    with pytest.raises(HostError):
        bm.schedule_prefill(100, [1], [(1, _tokens(2, 20))])  # waiting id already admitted
    with pytest.raises(HostError):
        bm.schedule_prefill(-1, [1], [])
    with pytest.raises(HostError):
        bm.schedule_prefill(100, [1, 1], [])  # an in-progress sequence listed twice
    with pytest.raises(HostError):
        bm.schedule_prefill(100, [], [(2, _tokens(2, 20)), (2, _tokens(3, 20))])  # a waiting id twice
    assert bm.free_blocks() == free
    bm.check_invariants()
