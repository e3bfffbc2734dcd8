"""End-to-end GPU scenarios at the shapes of the measurement configurations:
the host block manager drives the device pool through the C ABI, and every
phase is checked against the oracle (bit-exact for appends, copies and
gathers; within the attention tolerances for decode attention).

Every scenario passes its metadata in the engine's host form (u32 slots,
page tables held by the step's plan).

* C1, Qwen2.5-0.5B f32: bulk prompt append, then 64 decode steps of
  (append one token + gather + attention) over all 24 layers.
* C4, radix sharing at Qwen-7B head shapes (2 of 28 layers): 256 sequences
  fork one 4,100-token prefix (256 full blocks + a 4-token partial block),
  copy-on-write of the shared partial block on the first append (255 copies,
  the last holder writes in place), suffixes ~U{64..1024}, 32 decode steps,
  the shared-prefix step over the block manager's tables (equal to the plain
  attention), then a third of the sequences finish, LRU eviction frees 20%
  of the live blocks and the pool is compacted by batched block moves.
* C5, pool pressure at Qwen-7B head shapes (1 of 28 layers): the
  217,982-block pool of a 200 GB budget, 512 sequences with log-normal
  lengths (median 2,048, sigma 1, capped at 32,768); per step 8 sequences
  append a 512-token chunk and attend over it causally (extend attention),
  and all others decode one token.
"""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import DeviceKvPool, PoolDesc
from mitten_amd import workloads as wl
from mitten_amd.host import BlockManager
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _tokens(seed, n):
    return np.random.default_rng(seed).integers(0, 50_000, n).astype(np.uint32)


def _ctx_indptr(ctx):
    return np.concatenate([[0], np.cumsum(ctx)]).astype(np.int32)


def _sub_batch(indptr, ids, ctx, rows):
    """CSR tables of a subset of the batch's sequences."""
    tabs = [ids[indptr[r]:indptr[r + 1]] for r in rows]
    sub_ptr = np.concatenate([[0], np.cumsum([len(t) for t in tabs])]).astype(np.int32)
    return sub_ptr, np.concatenate(tabs).astype(np.int32), np.asarray([ctx[r] for r in rows], np.int32)


# --------------------------------------------------------------------- C1 ----

def _u32(a):
    return np.ascontiguousarray(a, np.uint32)


def test_c1_prompt_append_prefill_then_decode_gather_attention():
    """The configuration as stated: 8 prompts ~U{32..512}, then 64 decode
    steps of (append + gather + attention) over all 24 layers, driven by the
    block manager through the host-metadata entry points."""
    c = wl.CONFIGS["qwen2.5-0.5b"]
    L, Hq, Hkv, D = c["num_layers"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"]
    rng = wl.SplitMix64(wl.BASE_SEED + c["index"])
    B, steps = c["batch"], 64
    prompts = [rng.uniform_int(c["ctx_lo"], c["ctx_hi"]) for _ in range(B)]
    num_blocks = sum((p + steps + 15) // 16 for p in prompts) + 4
    desc = PoolDesc(L, Hkv, Hq, D, num_blocks, "f32")
    od = odesc(desc)
    bm = BlockManager(num_blocks)
    want = np.zeros(desc.shape, np.float32)
    with DeviceKvPool(desc) as pool:
        pool.write(want)
        # Bulk prompt append, all layers in one launch (admission order, LIFO pool).
        slots = []
        for s, p in enumerate(prompts):
            assert bm.admit(s, _tokens(s, p)) == 0
            sl, cow = bm.append(s, p)
            assert cow == []
            slots.append(sl)
        slots = np.concatenate(slots).astype(np.int32)
        k = normal(100, (L, slots.size, Hkv, D), "f32")
        v = normal(101, (L, slots.size, Hkv, D), "f32")
        pool.append_all_layers(to_device(k), to_device(v), _u32(slots))
        for layer in range(L):
            assert orc.append(od, want, layer, k[layer], v[layer], slots) == -1
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(want))
        # Prefill attention of the prompts (causal, whole prompt as the chunk),
        # first and last layer.
        indptr, ids, ctx = bm.batch(list(range(B)))
        q_indptr = np.concatenate([[0], np.cumsum(prompts)]).astype(np.int32)
        for layer in (0, L - 1):
            qp = normal(4000 + layer, (int(q_indptr[-1]), Hq, D), "f32")
            o = pool.extend_attention_host(layer, to_device(qp), prompts, ctx, _u32(indptr), _u32(ids))
            pool.check()
            ref = orc.extend_attention(od, want, layer, qp, q_indptr, indptr, ids, ctx)
            assert_attention_close(to_host(o), ref, "f32")
        plan = pool.plan(np.ones(B, np.int32))
        for step in range(steps):
            new = np.concatenate([bm.append(s, 1)[0] for s in range(B)]).astype(np.int32)
            indptr, ids, ctx = bm.batch(list(range(B)))
            assert np.array_equal(new, [ids[indptr[b] + (ctx[b] - 1) // 16] * 16 + (ctx[b] - 1) % 16
                                        for b in range(B)])
            plan.build(ctx, block_indptr=_u32(indptr), block_ids=_u32(ids))
            check_layers = range(L) if step in (0, steps - 1) else (0, L - 1)
            for layer in range(L):
                kn = normal(1000 + 31 * step + layer, (B, Hkv, D), "f32")
                vn = normal(2000 + 31 * step + layer, (B, Hkv, D), "f32")
                q = normal(3000 + 31 * step + layer, (B, Hq, D), "f32")
                o = pool.decode_step(layer, plan, to_device(kn), to_device(vn), to_device(q), None, None)
                gk, gv = pool.gather_host(layer, _u32(indptr), _u32(ids), ctx)
                assert orc.append(od, want, layer, kn, vn, new) == -1
                if layer in check_layers:
                    wk, wv = orc.gather(od, want, layer, indptr, ids, ctx)
                    assert np.array_equal(bits(to_host(gk)), bits(wk))
                    assert np.array_equal(bits(to_host(gv)), bits(wv))
                    ref = orc.decode_attention(od, want, layer, q, indptr, ids, ctx)
                    assert_attention_close(to_host(o), ref, "f32")
        plan.close()
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(want))
    bm.check_invariants()


# --------------------------------------------------------------------- C4 ----


def test_c4_radix_sharing_cow_decode_eviction_and_compaction():
    """The radix-sharing configuration at its stated size (2 of 28 layers at
    Qwen-7B heads): 256 sequences share a 4,100-token prefix (the partial
    block copied on write 255 times), suffixes ~U{64..1024}, 32 decode steps
    (the fused step over the block manager's tables; the shared-prefix step
    checked against it), then a third of the sequences finish, LRU eviction
    frees 20% of the live blocks, and the compaction's block moves pack the
    pool. Pool bit-exact against the oracle after every phase; the live
    sequences' gathers and attention bit-identical across the compaction."""
    L, Hq, Hkv, D = 2, 28, 4, 128
    sc = wl.RadixSharingScenario()
    bm, seqs = sc.bm, sc.seqs
    B = sc.num_seqs
    desc = PoolDesc(L, Hkv, Hq, D, sc.num_blocks, "bf16")
    od = odesc(desc)
    want = np.zeros(desc.shape, np.uint16)
    with DeviceKvPool(desc) as pool:
        pool.write(want)
        # 1. The prefix, prefilled once.
        pslots = sc.prefill_prefix()
        k = normal(200, (L, pslots.size, Hkv, D), "bf16")
        v = normal(201, (L, pslots.size, Hkv, D), "bf16")
        pool.append_all_layers(to_device(k), to_device(v), _u32(pslots))
        for layer in range(L):
            assert orc.append(od, want, layer, k[layer], v[layer], pslots) == -1
        shared = bm.table(0)
        # 2. Forks, copy-on-write of the shared partial block, suffixes.
        src, dst, slots = sc.fork_and_suffixes()
        assert len(src) == B - 1 and set(src.tolist()) == {int(shared[-1])}
        assert bm.table(0)[sc.prefix_full_blocks] == shared[-1]  # the last holder kept it
        assert all(bm.refcount(int(b)) == B + 1 for b in shared[:-1])  # every sequence + the tree
        pool.copy_blocks(_u32(src), _u32(dst))
        orc.copy_blocks(od, want, src, dst)
        k = normal(202, (L, slots.size, Hkv, D), "bf16")
        v = normal(203, (L, slots.size, Hkv, D), "bf16")
        pool.append_all_layers(to_device(k), to_device(v), _u32(slots))
        for layer in range(L):
            assert orc.append(od, want, layer, k[layer], v[layer], slots) == -1
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(want))
        bm.check_invariants()
        # 3. 32 decode steps over all 256 sequences.
        sample = list(range(0, B, 16))
        plan = pool.plan(np.ones(B, np.int32))
        for step in range(sc.decode_steps):
            new = sc.decode_step()
            indptr, ids, ctx = bm.batch(seqs)
            plan.build(ctx, block_indptr=_u32(indptr), block_ids=_u32(ids))
            for layer in range(L):
                kn = normal(300 + 7 * step + layer, (B, Hkv, D), "bf16")
                vn = normal(400 + 7 * step + layer, (B, Hkv, D), "bf16")
                q = normal(500 + 7 * step + layer, (B, Hq, D), "bf16")
                o = pool.decode_step(layer, plan, to_device(kn), to_device(vn), to_device(q), None, None)
                assert orc.append(od, want, layer, kn, vn, new) == -1
                if step % 8 == 7 or step == 0:
                    sp, si, sc_ = _sub_batch(indptr, ids, ctx, sample)
                    ref = orc.decode_attention(od, want, layer, widen(q[sample]), sp, si, sc_)
                    assert_attention_close(to_host(o)[sample], ref, "bf16")
        plan.close()
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(want))
        # The shared-prefix step over the same tables: the prefix's 256 full
        # pages read once for all 256 sequences, then each suffix.
        indptr, ids, ctx = bm.batch(seqs)
        pre, s_ptr, s_ids, s_len = bm.batch_shared_prefix(seqs)
        assert pre.size == sc.prefix_full_blocks and np.array_equal(pre, shared[:-1])
        q = normal(550, (B, Hq, D), "bf16")
        plan = pool.plan(ctx, block_indptr=_u32(indptr), block_ids=_u32(ids))
        o_full = to_host(pool.decode_attention_planned(1, plan, to_device(q), None, None))
        plan.close()
        splan = pool.plan_shared_prefix(_u32(pre), s_len, _u32(s_ptr), _u32(s_ids))
        o_sp = to_host(pool.decode_step_shared_prefix(1, splan, None, None, to_device(q), None, None, None))
        splan.close()
        pool.check()
        assert_attention_close(o_sp, widen(o_full), "bf16")
        sp_, si_, sc2 = _sub_batch(indptr, ids, ctx, sample)
        assert_attention_close(o_sp[sample], orc.decode_attention(od, want, 1, widen(q[sample]), sp_, si_, sc2),
                               "bf16")
        # 4. A third of the sequences finish; LRU eviction frees 20% of the blocks.
        live_tabs = {s: bm.table(s).copy() for s in seqs}
        done, freed, live_before = sc.finish_and_evict()
        live = sc.live
        assert freed >= 0.2 * live_before and bm.live_blocks() == live_before - freed
        bm.check_invariants()
        indptr, ids, ctx = bm.batch(live)
        assert all(np.array_equal(bm.table(s), live_tabs[s]) for s in live)
        before = [to_host(t) for t in pool.gather_host(0, _u32(indptr), _u32(ids), ctx)]
        q = normal(600, (len(live), Hq, D), "bf16")
        plan = pool.plan(ctx, block_indptr=_u32(indptr), block_ids=_u32(ids))
        o_before = to_host(pool.decode_attention_planned(1, plan, to_device(q), None, None))
        plan.close()
        # 5. Compaction: the moves pack the live blocks below the live count.
        src, dst = sc.compaction()
        assert len(src) > 0 and set(src.tolist()).isdisjoint(dst.tolist())
        pool.copy_blocks(_u32(src), _u32(dst))
        orc.copy_blocks(od, want, src, dst)
        bm.check_invariants()
        indptr2, ids2, ctx2 = bm.batch(live)
        assert np.array_equal(ctx2, ctx) and int(ids2.max()) < bm.live_blocks()
        after = [to_host(t) for t in pool.gather_host(0, _u32(indptr2), _u32(ids2), ctx2)]
        assert all(np.array_equal(bits(a), bits(b)) for a, b in zip(after, before))
        plan = pool.plan(ctx2, block_indptr=_u32(indptr2), block_ids=_u32(ids2))
        o_after = to_host(pool.decode_attention_planned(1, plan, to_device(q), None, None))
        plan.close()
        assert np.array_equal(bits(o_after), bits(o_before))  # same bytes, same order: same bits
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(want))


# --------------------------------------------------------------------- C5 ----

C5_BLOCKS, C5_SEQS, C5_CHUNK, C5_CHUNK_SEQS, C5_BUDGET = 217_982, 512, 512, 8, 4096


def test_c5_pool_pressure_chunked_append_and_decode():
    """Sixteen prefills in progress, each with a 512-token chunk of its prompt
    left; the block manager's budget rule (PrefillAdder, 4,096 prefill tokens
    per step) gives the first eight their chunks in the first step and the
    other eight in the second. Every sequence whose prefill is done decodes
    one token per step."""
    import torch

    L, Hq, Hkv, D = 1, 28, 4, 128  # Qwen-7B heads, 1 of 28 layers
    rng = wl.SplitMix64(wl.BASE_SEED + 4)
    lengths = wl.lognormal_lengths(rng, C5_SEQS, 2048, 1.0, 32768)
    desc = PoolDesc(L, Hkv, Hq, D, C5_BLOCKS, "bf16")
    bm = BlockManager(C5_BLOCKS)
    seqs = list(range(C5_SEQS))
    prefilling = seqs[:2 * C5_CHUNK_SEQS]
    prompt = [n + (C5_CHUNK if s in prefilling else 0) for s, n in enumerate(lengths)]
    for s in seqs:
        bm.admit(s, _tokens(10_000 + s, prompt[s]))
        bm.append(s, lengths[s])
    assert bm.live_blocks() == sum((n + 15) // 16 for n in prompt)
    with DeviceKvPool(desc) as pool:
        view = pool.tensor()
        gen = torch.Generator(device="cuda")
        gen.manual_seed(5)
        view.normal_(generator=gen)  # every slot holds N(0,1) K/V
        torch.cuda.synchronize()

        def blocks_of(table):
            """Host copy of the given blocks of layer 0: [2, n, 16, Hkv, D] bf16 bits."""
            t = view[0][:, torch.from_numpy(np.asarray(table, np.int64)).cuda()]
            return to_host(t.contiguous())

        for step in range(2):
            got, _, _, _ = bm.schedule_prefill(C5_BUDGET, prefilling, [])
            chunk = [s for s, c in zip(prefilling, got) if c]
            assert chunk == seqs[step * C5_CHUNK_SEQS:(step + 1) * C5_CHUNK_SEQS]
            assert [c for c in got if c] == [C5_CHUNK] * C5_CHUNK_SEQS
            slots = np.concatenate([bm.append(s, C5_CHUNK)[0] for s in chunk]).astype(np.int32)
            kc = normal(700 + step, (slots.size, Hkv, D), "bf16")
            vc = normal(800 + step, (slots.size, Hkv, D), "bf16")
            pool.append(0, to_device(kc), to_device(vc), _u32(slots))
            blk = torch.from_numpy((slots // 16).astype(np.int64)).cuda()
            off = torch.from_numpy((slots % 16).astype(np.int64)).cuda()
            assert np.array_equal(to_host(view[0, 0, blk, off]), kc)
            assert np.array_equal(to_host(view[0, 1, blk, off]), vc)
            # The chunks' causal attention over their whole caches (extend).
            cptr, cids, cctx = bm.batch(chunk)
            qc = normal(850 + step, (len(chunk) * C5_CHUNK, Hq, D), "bf16")
            oc = to_host(pool.extend_attention_host(0, to_device(qc), [C5_CHUNK] * len(chunk), cctx, _u32(cptr),
                                                    _u32(cids)))
            for r in (0, len(chunk) - 1):  # two chunk sequences, first / middle / last queries
                table = cids[cptr[r]:cptr[r + 1]]
                mini = np.ascontiguousarray(blocks_of(table)[None])
                md = orc.desc(1, Hkv, D, len(table), 2)
                rows = [0, 1, C5_CHUNK // 2, C5_CHUNK - 1]
                pos = [int(cctx[r]) - C5_CHUNK + i for i in rows]
                need = [p // 16 + 1 for p in pos]
                vptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
                vids = np.concatenate([np.arange(k, dtype=np.int32) for k in need])
                ref = orc.decode_attention(md, mini, 0, widen(qc[[r * C5_CHUNK + i for i in rows]]), vptr, vids,
                                           np.asarray([p + 1 for p in pos], np.int32))
                assert_attention_close(oc[[r * C5_CHUNK + i for i in rows]], ref, "bf16")
            dec = [s for s in seqs if s not in prefilling]  # prefill done: decoding
            prefilling = [s for s in prefilling if s not in chunk]  # these chunks end their prompts
            new = np.concatenate([bm.append(s, 1)[0] for s in dec]).astype(np.int32)
            indptr, ids, ctx = bm.batch(dec)
            plan = pool.plan(ctx, block_indptr=_u32(indptr), block_ids=_u32(ids))
            kn = normal(900 + step, (len(dec), Hkv, D), "bf16")
            vn = normal(950 + step, (len(dec), Hkv, D), "bf16")
            q = normal(990 + step, (len(dec), Hq, D), "bf16")
            o = to_host(pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), None, None))
            plan.close()
            pool.check()
            blk = torch.from_numpy((new // 16).astype(np.int64)).cuda()
            off = torch.from_numpy((new % 16).astype(np.int64)).cuda()
            assert np.array_equal(to_host(view[0, 0, blk, off]), kn)  # fused append, bit-exact
            assert np.array_equal(to_host(view[0, 1, blk, off]), vn)
            # Attention of a sample (short, median and the longest sequences)
            # against the oracle over those sequences' blocks.
            order = np.argsort(ctx)
            sample = sorted(set(order[:4].tolist() + order[len(order) // 2:len(order) // 2 + 4].tolist()
                                + order[-8:].tolist()))
            for r in sample:
                table = ids[indptr[r]:indptr[r + 1]]
                mini = blocks_of(table)[None]  # [1, 2, n, 16, Hkv, D]
                md = orc.desc(1, Hkv, D, len(table), 2)
                ref = orc.decode_attention(md, np.ascontiguousarray(mini), 0, widen(q[r:r + 1]),
                                           np.array([0, len(table)], np.int32),
                                           np.arange(len(table), dtype=np.int32), ctx[r:r + 1])
                assert_attention_close(o[r:r + 1], ref, "bf16")
        del view
    bm.check_invariants()
