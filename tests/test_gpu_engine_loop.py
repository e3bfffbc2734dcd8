"""An engine loop on the GPU, the way the engine's scheduler and a paged
backend drive the path step by step (inference-engine/src/scheduler.rs:8-77,
prefill.rs:21-114, decode.rs:6-47; the calls the Rust PagedLifecycle and
PagedBackend make):

* each step's prefill budget is max_prefill_tokens_per_iter minus the decode
  tokens (scheduler.rs:14-18); the host block manager's budget rule schedules
  the in-progress prefills first, then admits waiting prompts (radix prefix
  hits included) while budget remains;
* the step's writes get their slots from the block manager (a shared block
  about to be written is copied first: forks for parallel sampling);
* per layer, prefill chunks append their K/V (host slots) and run causal
  extend attention over their whole caches (host tables), and decode tokens
  run the fused append + attention from a plan holding the step's tables;
* a finished prefill is promoted into the radix tree and starts decoding;
  a finished request releases its blocks; LRU eviction and compaction move
  blocks when the pool runs short and every fifth step.

A host mirror of the pool receives the same appends and block copies through
the oracle. Every attention output of every step is checked against the
oracle over the mirror, every step's block books against their invariants,
and the device pool against the mirror bit for bit at the end."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import DeviceKvPool, PoolDesc
from mitten_amd.host import BlockManager
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

SHAPES = {
    # name: (layers, Hq, Hkv, D, dtype)
    "qwen0.5b-f32": (2, 14, 2, 64, "f32"),
    "qwen7b-bf16": (2, 28, 4, 128, "bf16"),
}


class Req:
    def __init__(self, seq, prompt, max_new):
        self.seq, self.prompt, self.max_new = seq, prompt, max_new
        self.generated = 0


def _u32(a):
    return np.ascontiguousarray(a, np.uint32)


@pytest.mark.parametrize("shape", list(SHAPES))
def test_engine_loop_matches_the_oracle_every_step(shape):
    L, Hq, Hkv, D, dt = SHAPES[shape]
    num_blocks, max_prefill = 72, 48
    desc = PoolDesc(L, Hkv, Hq, D, num_blocks, dt)
    od = odesc(desc)
    rng = np.random.default_rng(2026)
    shared = rng.integers(0, 50_000, 40).astype(np.uint32)  # a common 40-token prefix (2 full pages)
    waiting = []
    for s in range(12):
        own = rng.integers(0, 50_000, int(rng.integers(5, 60))).astype(np.uint32)
        prompt = np.concatenate([shared, own]) if s % 2 == 0 else own
        waiting.append(Req(s + 1, prompt, int(rng.integers(2, 7))))
    bm = BlockManager(num_blocks, 16, max_cached_pages=24)
    mirror = normal(1, desc.shape, dt)
    prefilling, decoding, done = [], [], []
    next_seq, seed = 1000, 10
    hits = forks = cow_copies = moves = 0
    with DeviceKvPool(desc) as pool:
        pool.write(mirror)

        def copy(src, dst):
            pool.copy_blocks(_u32(src), _u32(dst))
            orc.copy_blocks(od, mirror, np.asarray(src, np.int32), np.asarray(dst, np.int32))

        for step in range(200):
            if not (waiting or prefilling or decoding):
                break
            # Schedule (scheduler.rs:8-27): decode requests, then prefill chunks under the budget.
            budget = max(0, max_prefill - len(decoding))
            in_prog = list(prefilling)
            ip, wc, n_adm, cached = bm.schedule_prefill(budget, [r.seq for r in in_prog],
                                                        [(r.seq, r.prompt) for r in waiting])
            admitted, waiting = waiting[:n_adm], waiting[n_adm:]
            hits += sum(1 for c in cached if c > 0)
            prefilling = in_prog + admitted
            chunks = [(r, c) for r, c in zip(prefilling, ip + wc[:n_adm]) if c > 0]
            decode = list(decoding)
            # Slots of the step's writes; copy-on-write pairs run before the appends.
            src, dst, pre_slots, dec_slots = [], [], [], []
            for r, c in chunks:
                slots, cow = bm.append(r.seq, c)
                pre_slots.append(slots)
                for s_, d_ in cow:
                    src.append(s_)
                    dst.append(d_)
            for r in decode:
                slots, cow = bm.append(r.seq, 1)
                dec_slots.append(int(slots[0]))
                for s_, d_ in cow:
                    src.append(s_)
                    dst.append(d_)
            if src:
                copy(src, dst)
                cow_copies += len(src)
            plan = None
            if decode:
                dptr, dids, dctx = bm.batch([r.seq for r in decode])
                plan = pool.plan(dctx, block_indptr=_u32(dptr), block_ids=_u32(dids))
            if chunks:
                pptr, pids, pctx = bm.batch([r.seq for r, _ in chunks])
                qlens = [c for _, c in chunks]
                qptr = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
                slots_all = np.concatenate(pre_slots).astype(np.int32)
            for layer in range(L):
                if chunks:
                    T = int(qptr[-1])
                    k, v = normal(seed, (T, Hkv, D), dt), normal(seed + 1, (T, Hkv, D), dt)
                    q = normal(seed + 2, (T, Hq, D), dt)
                    seed += 3
                    pool.append(layer, to_device(k), to_device(v), _u32(slots_all))
                    orc.append(od, mirror, layer, k, v, slots_all)
                    o = to_host(pool.extend_attention_host(layer, to_device(q), qlens, pctx, _u32(pptr),
                                                           _u32(pids)))
                    ref = orc.extend_attention(od, mirror, layer, widen(q), qptr, pptr, pids, pctx)
                    assert_attention_close(o, ref, dt)
                if decode:
                    B = len(decode)
                    kn, vn, q = normal(seed, (B, Hkv, D), dt), normal(seed + 1, (B, Hkv, D), dt), \
                        normal(seed + 2, (B, Hq, D), dt)
                    seed += 3
                    o = to_host(pool.decode_step(layer, plan, to_device(kn), to_device(vn), to_device(q), None,
                                                 None))
                    orc.append(od, mirror, layer, kn, vn, np.asarray(dec_slots, np.int32))
                    ref = orc.decode_attention(od, mirror, layer, widen(q), dptr, dids, dctx)
                    assert_attention_close(o, ref, dt)
            if plan is not None:
                plan.close()
            pool.check()
            # Transitions (scheduler.rs:88-179): finished prefills are promoted
            # and decode (every third one forks a sibling for parallel sampling);
            # finished decodes release their blocks.
            for r, _ in chunks:
                if bm.seq_len(r.seq) == r.prompt.size:
                    prefilling.remove(r)
                    bm.promote(r.seq, r.prompt)
                    decoding.append(r)
                    if r.seq % 3 == 0:
                        bm.fork(r.seq, next_seq)
                        decoding.append(Req(next_seq, r.prompt, r.max_new))
                        next_seq += 1
                        forks += 1
            for r in decode:
                r.generated += 1
                if r.generated >= r.max_new:
                    decoding.remove(r)
                    bm.release(r.seq)
                    done.append(r)
            # Pool upkeep: when the pool runs short, and every fifth step
            # after releases leave holes, evict cached pages and pack the
            # live blocks below the live count.
            if bm.free_blocks() < 16 or step % 5 == 4:
                bm.evict(8)
                s_, d_ = bm.plan_compaction()
                if s_.size:
                    copy(s_, d_)
                    moves += int(s_.size)
            bm.check_invariants()
        assert not (waiting or prefilling or decoding), "the loop did not drain"
        assert np.array_equal(bits(pool.read()), bits(mirror))
    # Every lifecycle event happened at least once.
    assert len(done) == 12 + forks
    assert hits > 0 and forks > 0 and cow_copies > 0 and moves > 0, (hits, forks, cow_copies, moves)
