"""CPU checks of the seeded measurement workloads: the shared-prefix decode
batch and the pool-pressure step hold the invariants their configurations
state, each checked from the tables themselves."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import workloads as wl


def _tables(batch):
    return [batch.block_ids[batch.block_indptr[b]:batch.block_indptr[b + 1]] for b in range(batch.num_seqs)]


def _check_slots(batch, positions):
    for b, t in enumerate(_tables(batch)):
        p = int(positions[b])
        assert batch.slot_mapping[b] == t[p // 16] * 16 + p % 16


def test_shared_prefix_batch_shares_full_prefix_blocks_only():
    seqs, prefix = 40, 4100
    b = wl.shared_prefix_batch(seqs, prefix, 64, 1024, wl.SplitMix64(11))
    tabs = _tables(b)
    full = prefix // 16  # 256 full blocks; the 4-token partial block is per sequence (after COW)
    shared = tabs[0][:full]
    assert all(np.array_equal(t[:full], shared) for t in tabs)
    own = np.concatenate([t[full:] for t in tabs])
    assert np.unique(own).size == own.size and not np.isin(own, shared).any()
    assert np.array_equal(b.meta["own_first"], [t[full] for t in tabs])
    # every table covers its context; ids form a permutation of the pool
    assert all(len(t) == (c + 15) // 16 for t, c in zip(tabs, b.ctx_lens))
    assert np.array_equal(np.sort(np.concatenate([shared, own])), np.arange(b.num_blocks))
    assert all(prefix + 64 + 1 <= c <= prefix + 1024 + 1 for c in b.ctx_lens)
    _check_slots(b, b.ctx_lens - 1)  # the appended token sits at position ctx - 1
    # unique tokens: distinct (block, row) positions attended
    seen = set()
    for t, c in zip(tabs, b.ctx_lens):
        seen.update((int(t[p // 16]), p % 16) for p in range(int(c)))
    assert b.meta["unique_tokens"] == len(seen)


def test_pool_pressure_step_tables_chunks_and_lengths():
    nblocks, seqs, chunk, cs = 60_000, 64, 512, 8
    batch, chunk_slots, lengths = wl.pool_pressure_step(nblocks, seqs, chunk, cs, wl.SplitMix64(12))
    assert lengths.size == seqs and lengths.min() >= 1 and lengths.max() <= 32768
    assert batch.num_seqs == seqs - cs
    assert np.array_equal(batch.ctx_lens, lengths[cs:] + 1)
    _check_slots(batch, lengths[cs:])
    # chunk slots: distinct, inside the pool, never a decode sequence's block
    assert chunk_slots.size == cs * chunk and np.unique(chunk_slots).size == chunk_slots.size
    assert chunk_slots.min() >= 0 and chunk_slots.max() < nblocks * 16
    assert not np.isin(np.unique(chunk_slots // 16), batch.block_ids).any()
    ids = batch.block_ids
    assert np.unique(ids).size == ids.size and ids.max() < nblocks


def test_lognormal_lengths_median_and_cap():
    x = np.asarray(wl.lognormal_lengths(wl.SplitMix64(13), 4000, 2048, 1.0, 32768))
    assert x.min() >= 1 and x.max() <= 32768
    assert 1800 < np.median(x) < 2300  # median of LogNormal(ln 2048, 1)
    lx = np.log(x[(x > 1) & (x < 32768)])
    assert 0.9 < lx.std() < 1.1


def test_pool_pressure_chunks_come_from_the_budget_rule():
    """The chunks are the budget rule's: 8 prefills with 512 tokens left fill a
    4,096-token budget; at 4,000 the eighth gets the 416 tokens left; a
    budget that leaves a prefill without a chunk this step is refused (that
    prefill would neither prefill nor decode)."""
    batch, chunk_slots, _ = wl.pool_pressure_step(60_000, 64, 512, 8, wl.SplitMix64(12), budget=4096)
    assert chunk_slots.size == 8 * 512
    _, short, _ = wl.pool_pressure_step(60_000, 64, 512, 8, wl.SplitMix64(12), budget=4000)
    assert short.size == 7 * 512 + 416
    assert np.array_equal(short, chunk_slots[:short.size])  # the same slots, the last chunk cut short
    with pytest.raises(ValueError):
        wl.pool_pressure_step(60_000, 64, 512, 8, wl.SplitMix64(12), budget=7 * 512)
