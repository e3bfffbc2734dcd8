"""GPU parity of the host-metadata entry points (the engine's u32 form):
page tables as host CSR, slots and copy pairs as host u32 arrays, validated
on the host and copied by the library before the call returns
(inference-backend/src/batch.rs:24-26, inference-engine/src/request.rs:6).
Every result is compared with the oracle and with the device-array entry
point on the same inputs; plans that hold their tables are compared with
plans whose calls bring device tables. Device tables rewritten in place
between calls must be seen by the next call."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import BackendError, DeviceKvPool, PoolDesc
from mitten_amd import device_pool as dp
from mitten_amd import workloads as wl
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

SHAPES = {
    # name: (layers, Hq, Hkv, D, dtype)
    "qwen0.5b-f32": (2, 14, 2, 64, "f32"),
    "qwen7b-bf16": (2, 28, 4, 128, "bf16"),
    "gemma2b-bf16": (2, 8, 1, 256, "bf16"),
    "llama8b-bf16": (1, 32, 8, 128, "bf16"),
}


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _pool(shape, num_blocks, seed):
    L, Hq, Hkv, D, dt = SHAPES[shape]
    desc = PoolDesc(L, Hkv, Hq, D, num_blocks, dt)
    pool = DeviceKvPool(desc)
    host = normal(seed, desc.shape, dt)
    pool.write(host)
    return desc, pool, host


@pytest.mark.parametrize("shape", list(SHAPES))
def test_append_host_bit_exact_and_copied_before_return(shape):
    """The slots are u32 host values; the caller overwrites its array right
    after the call returns, before the stream runs, and the pool still gets
    the original slots."""
    import torch

    desc, pool, host = _pool(shape, 40, 1)
    n = 37
    slots = np.random.default_rng(2).choice(desc.num_blocks * 16, size=n, replace=False).astype(np.uint32)
    k = normal(3, (n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(4, (n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    layer = desc.num_layers - 1
    mine = slots.copy()
    torch.cuda._sleep(2_000_000)  # keep the stream busy so the upload runs after the overwrite below
    pool.append(layer, to_device(k), to_device(v), mine)
    mine[:] = 0
    pool.check()
    want = host.copy()
    assert orc.append(odesc(desc), want, layer, k, v, slots.astype(np.int32)) == -1
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


def test_append_all_layers_host_bit_exact():
    desc, pool, host = _pool("qwen7b-bf16", 24, 5)
    n = 50
    slots = np.random.default_rng(6).choice(desc.num_blocks * 16, size=n, replace=False).astype(np.uint32)
    k = normal(7, (desc.num_layers, n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(8, (desc.num_layers, n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    pool.append_all_layers(to_device(k), to_device(v), slots)
    pool.check()
    want = host.copy()
    for layer in range(desc.num_layers):
        orc.append(odesc(desc), want, layer, np.ascontiguousarray(k[layer]), np.ascontiguousarray(v[layer]),
                   slots.astype(np.int32))
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


def test_append_host_bad_slot_rejected_before_launch():
    """An out-of-range slot is an argument error on the host: nothing is
    written, not even the valid rows, and the device error word stays clear."""
    desc, pool, host = _pool("qwen7b-bf16", 8, 9)
    k = normal(10, (3, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(11, (3, desc.num_kv_heads, desc.head_dim), desc.dtype)
    with pytest.raises(BackendError) as ei:
        pool.append(0, to_device(k), to_device(v), np.array([3, desc.num_blocks * 16, 17], np.uint32))
    assert ei.value.status == dp.MKV_ERR_INVALID_ARGUMENT
    assert "slot[1]" in str(ei.value)
    pool.check()
    assert np.array_equal(bits(pool.read()), bits(host))
    pool.close()


@pytest.mark.parametrize("shape", ["qwen0.5b-f32", "qwen7b-bf16", "gemma2b-bf16"])
def test_gather_host_matches_device_form_and_oracle(shape):
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(12)
    batch = wl.decode_batch_from_contexts([0, 15, 16, 40, 300, 7], rng, extra_blocks=4)
    desc, pool, host = _pool(shape, batch.num_blocks, 13)
    layer = L - 1
    kh, vh = pool.gather_host(layer, batch.block_indptr.astype(np.uint32), batch.block_ids.astype(np.uint32),
                              batch.ctx_lens)
    kd, vd = pool.gather(layer, _i32(batch.block_indptr), _i32(batch.block_ids), _i32(batch.ctx_indptr),
                         batch.max_ctx)
    pool.check()
    assert np.array_equal(bits(to_host(kh)), bits(to_host(kd)))
    assert np.array_equal(bits(to_host(vh)), bits(to_host(vd)))
    wk, wv = orc.gather(odesc(desc), host, layer, batch.block_indptr, batch.block_ids, batch.ctx_lens)
    assert np.array_equal(bits(to_host(kh)), bits(wk))
    assert np.array_equal(bits(to_host(vh)), bits(wv))
    pool.close()


def test_host_ids_of_2_pow_32_or_more_are_refused_not_wrapped():
    """A slot of 2^32 + 5 would wrap to slot 5 in a u32 cast (a valid slot of
    the pool); a block id of 2^32 + 1 to block 1. Both are refused before
    anything is launched, and the pool is untouched."""
    desc, pool, host = _pool("qwen7b-bf16", 8, 14)
    k = normal(15, (2, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(16, (2, desc.num_kv_heads, desc.head_dim), desc.dtype)
    with pytest.raises(BackendError) as ei:
        pool.append(0, to_device(k), to_device(v), np.array([3, 2**32 + 5], np.int64))
    assert "2^32" in str(ei.value)
    with pytest.raises(BackendError) as ei:
        pool.plan([20], block_indptr=np.array([0, 2], np.int64), block_ids=np.array([0, 2**32 + 1], np.int64))
    assert "2^32" in str(ei.value)
    pool.check()
    assert np.array_equal(bits(pool.read()), bits(host))
    pool.close()


def test_gather_host_rejects_short_table():
    desc, pool, host = _pool("qwen7b-bf16", 8, 14)
    with pytest.raises(BackendError) as ei:
        pool.gather_host(0, np.array([0, 1], np.uint32), np.array([2], np.uint32), [17])
    assert "cannot hold" in str(ei.value)
    pool.close()


@pytest.mark.parametrize("shape", ["qwen0.5b-f32", "qwen7b-bf16"])
def test_copy_blocks_host_bit_exact(shape):
    desc, pool, host = _pool(shape, 30, 15)
    src = np.array([1, 2, 3, 29], np.uint32)
    dst = np.array([10, 0, 20, 4], np.uint32)
    pool.copy_blocks(src, dst)
    pool.check()
    want = host.copy()
    orc.copy_blocks(odesc(desc), want, src.astype(np.int32), dst.astype(np.int32))
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


@pytest.mark.parametrize("src,dst,msg", [([1, 2], [3, 3], "repeats"), ([1, 2], [2, 5], "both a source"),
                                         ([1, 30], [4, 5], "outside the pool")])
def test_copy_blocks_host_rejects_bad_pairs(src, dst, msg):
    desc, pool, host = _pool("qwen7b-bf16", 30, 16)
    with pytest.raises(BackendError) as ei:
        pool.copy_blocks(np.array(src, np.uint32), np.array(dst, np.uint32))
    assert msg in str(ei.value)
    pool.check()
    assert np.array_equal(bits(pool.read()), bits(host))
    pool.close()


PLAN_CTX = [1, 2, 15, 16, 17, 33, 100, 129, 257, 500, 1000, 3, 64, 65, 700]
PLANNED_KERNELS = [("qwen0.5b-f32", None), ("qwen7b-bf16", "mfma"), ("qwen7b-bf16", "mfma-per-head"),
                   ("qwen7b-bf16", "valu"), ("gemma2b-bf16", "mfma"), ("llama8b-bf16", "mfma")]


@pytest.mark.parametrize("pieces", [0, 7])
@pytest.mark.parametrize("shape,kernel", PLANNED_KERNELS)
def test_plan_with_host_tables_equals_device_tables(shape, kernel, pieces):
    """A plan built with the batch's host tables (mkv_decode_plan_build_tables)
    and calls without tables give bit-identical outputs and pools to a plan
    whose calls bring device tables, and match the oracle. The host tables
    are padded past ceil(ctx/16) like the engine's growing tables."""
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(20)
    batch = wl.decode_batch_from_contexts([c - 1 for c in PLAN_CTX], rng, extra_blocks=40)
    # one spare id at the end of every table, as a table with a block allocated ahead
    nb = np.diff(batch.block_indptr)
    used = set(batch.block_ids.tolist())
    spare = np.array([i for i in range(batch.num_blocks) if i not in used][:batch.num_seqs], np.int32)
    ip = np.zeros(batch.num_seqs + 1, np.uint32)
    np.cumsum(nb + 1, out=ip[1:])
    ids = np.concatenate([np.append(batch.block_ids[batch.block_indptr[b]:batch.block_indptr[b + 1]], spare[b])
                          for b in range(batch.num_seqs)]).astype(np.uint32)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    B = batch.num_seqs
    host = normal(21, desc.shape, dt)
    q, kn, vn = normal(22, (B, Hq, D), dt), normal(23, (B, Hkv, D), dt), normal(24, (B, Hkv, D), dt)
    res = []
    for held in (False, True):
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            if held:
                plan = pool.plan(batch.ctx_lens, pieces=pieces, block_indptr=ip, block_ids=ids)
                tabs = (None, None)
            else:
                plan = pool.plan(batch.ctx_lens, pieces=pieces)
                tabs = (_i32(ip.astype(np.int32)), _i32(ids.astype(np.int32)))
            o = pool.decode_step(L - 1, plan, to_device(kn), to_device(vn), to_device(q), *tabs, kernel=kernel)
            o2 = pool.decode_attention_planned(0, plan, to_device(q), *tabs, kernel=kernel)
            pool.check()
            res.append((to_host(o), to_host(o2), pool.read()))
            plan.close()
    for a, b in zip(res[0], res[1]):
        assert np.array_equal(bits(a), bits(b))
    want = host.copy()
    assert orc.append(odesc(desc), want, L - 1, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(res[1][2]), bits(want))
    ref = orc.decode_attention(odesc(desc), want, L - 1, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens)
    assert_attention_close(res[1][0], ref, dt)
    ref0 = orc.decode_attention(odesc(desc), want, 0, widen(q), batch.block_indptr, batch.block_ids,
                                batch.ctx_lens)
    assert_attention_close(res[1][1], ref0, dt)


@pytest.mark.parametrize("ip,ids,ctx,msg", [
    ([0, 2], [1, 99], [20], "outside the pool"),
    ([0, 1], [1], [20], "cannot hold"),
    ([1, 2], [1, 2], [5], "block_indptr[0]"),
    ([0, 2], [1, 2], [0], "< 1"),
    # An entry that falls back is refused before any id is read: sequence 0's
    # 38 blocks would otherwise be read past the 2 ids given.
    ([0, 40, 2], [1, 2], [600, 20], "not monotone at 1"),
])
def test_plan_host_tables_rejected(ip, ids, ctx, msg):
    desc = PoolDesc(1, 4, 28, 128, 10, "bf16")
    with DeviceKvPool(desc) as pool:
        with pytest.raises(BackendError) as ei:
            pool.plan(ctx, block_indptr=np.array(ip, np.uint32), block_ids=np.array(ids, np.uint32))
        assert ei.value.status == dp.MKV_ERR_INVALID_ARGUMENT
        assert msg in str(ei.value)


def test_plan_without_tables_needs_device_tables():
    desc = PoolDesc(1, 4, 28, 128, 10, "bf16")
    q = normal(25, (1, 28, 128), "bf16")
    with DeviceKvPool(desc) as pool:
        plan = pool.plan([20])
        with pytest.raises(BackendError) as ei:
            pool.decode_attention_planned(0, plan, to_device(q), None, None)
        assert "no tables" in str(ei.value)
        plan.close()


@pytest.mark.parametrize("shape,kernel", [("qwen7b-bf16", "mfma"), ("qwen7b-bf16", "mfma-per-head"),
                                          ("qwen0.5b-f32", None), ("gemma2b-bf16", "mfma")])
def test_device_tables_rewritten_in_place_are_followed(shape, kernel):
    """One plan, the same device table tensors on two calls: between them the
    caller rewrites the ids in place (as after copy-on-write or compaction).
    The second call must attend over the new blocks, whose contents differ."""
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(26)
    ctx = [40, 300, 17, 129, 1000]
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng, extra_blocks=120)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    B = batch.num_seqs
    host = normal(27, desc.shape, dt)
    q = normal(28, (B, Hq, D), dt)
    used = set(batch.block_ids.tolist())
    free = np.array([i for i in range(batch.num_blocks) if i not in used], np.int32)
    ids2 = batch.block_ids.copy()
    ids2[::2] = free[:ids2[::2].size]  # every other block now points at another block's (different) data
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan(batch.ctx_lens, pieces=6)
        ip, ix = _i32(batch.block_indptr), _i32(batch.block_ids)
        o1 = to_host(pool.decode_attention_planned(0, plan, to_device(q), ip, ix, kernel=kernel))
        ix.copy_(_i32(ids2))  # same tensor, same address, new contents
        o2 = to_host(pool.decode_attention_planned(0, plan, to_device(q), ip, ix, kernel=kernel))
        pool.check()
        plan.close()
    r1 = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens)
    r2 = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, ids2, batch.ctx_lens)
    assert_attention_close(o1, r1, dt)
    assert_attention_close(o2, r2, dt)
    assert np.max(np.abs(r1 - r2)) > 0.05  # the two tables really give different results


@pytest.mark.parametrize("shape,kernel", [("qwen7b-bf16", "mfma"), ("qwen7b-bf16", "mfma-per-head"),
                                          ("qwen0.5b-f32", None), ("gemma2b-bf16", "mfma")])
def test_held_tables_survive_a_call_with_device_tables(shape, kernel):
    """A plan holding its build-time tables, called first without tables, then
    with device tables that point elsewhere, then without tables again: the
    third call attends over the build-time tables, bit-identical to the
    first, and the second over the device tables."""
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(29)
    ctx = [40, 300, 17, 129, 1000]
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng, extra_blocks=120)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    B = batch.num_seqs
    host = normal(35, desc.shape, dt)
    q = normal(36, (B, Hq, D), dt)
    used = set(batch.block_ids.tolist())
    free = np.array([i for i in range(batch.num_blocks) if i not in used], np.int32)
    ids2 = batch.block_ids.copy()
    ids2[::2] = free[:ids2[::2].size]
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan(batch.ctx_lens, pieces=6, block_indptr=batch.block_indptr.astype(np.uint32),
                         block_ids=batch.block_ids.astype(np.uint32))
        qd = to_device(q)
        o_held = to_host(pool.decode_attention_planned(0, plan, qd, None, None, kernel=kernel))
        o_dev = to_host(pool.decode_attention_planned(0, plan, qd, _i32(batch.block_indptr), _i32(ids2),
                                                      kernel=kernel))
        o_again = to_host(pool.decode_attention_planned(0, plan, qd, None, None, kernel=kernel))
        pool.check()
        plan.close()
    assert np.array_equal(bits(o_again), bits(o_held))
    r1 = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens)
    r2 = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, ids2, batch.ctx_lens)
    assert_attention_close(o_held, r1, dt)
    assert_attention_close(o_dev, r2, dt)
    assert np.max(np.abs(r1 - r2)) > 0.05  # the two tables really give different results


@pytest.mark.parametrize("shape", ["qwen7b-bf16", "gemma2b-bf16"])
def test_shared_prefix_plan_with_host_tables(shape):
    """plan_shared_prefix (prefix ids and suffix tables held by the plan)
    gives bit-identical outputs and pools to the device-table form."""
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(30)
    prefix_blocks, B = 9, 13
    suffix = np.array([rng.uniform_int(1, 200) for _ in range(B)], np.int32)
    nb = (suffix + 15) // 16
    num_blocks = prefix_blocks + int(nb.sum()) + 5
    perm = wl.permutation(num_blocks, rng)
    prefix = perm[:prefix_blocks]
    ip = np.zeros(B + 1, np.int32)
    np.cumsum(nb, out=ip[1:])
    ids = perm[prefix_blocks:prefix_blocks + int(nb.sum())]
    desc = PoolDesc(L, Hkv, Hq, D, num_blocks, dt)
    host = normal(31, desc.shape, dt)
    q, kn, vn = normal(32, (B, Hq, D), dt), normal(33, (B, Hkv, D), dt), normal(34, (B, Hkv, D), dt)
    res = []
    for held in (False, True):
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            if held:
                plan = pool.plan_shared_prefix(prefix.astype(np.uint32), suffix, ip.astype(np.uint32),
                                               ids.astype(np.uint32), pieces=5)
                o = pool.decode_step_shared_prefix(1, plan, to_device(kn), to_device(vn), to_device(q), None,
                                                   None, None)
            else:
                plan = pool.plan_suffixes(suffix, pieces=5)
                o = pool.decode_step_shared_prefix(1, plan, to_device(kn), to_device(vn), to_device(q),
                                                   _i32(prefix), _i32(ip), _i32(ids))
            pool.check()
            res.append((to_host(o), pool.read()))
            plan.close()
    assert np.array_equal(bits(res[0][0]), bits(res[1][0]))
    assert np.array_equal(bits(res[0][1]), bits(res[1][1]))
    full_ip = np.zeros(B + 1, np.int32)
    np.cumsum(nb + prefix_blocks, out=full_ip[1:])
    full_ids = np.concatenate([np.concatenate([prefix, ids[ip[b]:ip[b + 1]]]) for b in range(B)]).astype(np.int32)
    ctx = (prefix_blocks * 16 + suffix).astype(np.int32)
    want = host.copy()
    pos = ctx - 1
    slots = full_ids[full_ip[:-1] + pos // 16].astype(np.int64) * 16 + pos % 16
    assert orc.append(odesc(desc), want, 1, kn, vn, slots.astype(np.int32)) == -1
    assert np.array_equal(bits(res[1][1]), bits(want))
    ref = orc.decode_attention(odesc(desc), want, 1, widen(q), full_ip, full_ids, ctx)
    assert_attention_close(res[1][0], ref, dt)


@pytest.mark.parametrize("shape", ["qwen0.5b-f32", "qwen7b-bf16", "gemma2b-bf16"])
def test_extend_host_equals_device_form(shape):
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(40)
    ctx = np.array([70, 300, 16, 1, 520], np.int32)
    ql = np.array([20, 64, 16, 1, 0], np.int32)
    batch = wl.decode_batch_from_contexts(list(ctx - 1), rng, extra_blocks=3)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    host = normal(41, desc.shape, dt)
    T = int(ql.sum())
    q = normal(42, (T, Hq, D), dt)
    qip = np.zeros(ctx.size + 1, np.int32)
    np.cumsum(ql, out=qip[1:])
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        oh = to_host(pool.extend_attention_host(0, to_device(q), ql, ctx, batch.block_indptr.astype(np.uint32),
                                                batch.block_ids.astype(np.uint32)))
        od = to_host(pool.extend_attention(0, to_device(q), _i32(qip), _i32(batch.block_indptr),
                                           _i32(batch.block_ids), _i32(ctx), int(ql.max()), int(ctx.max())))
        pool.check()
    assert np.array_equal(bits(oh), bits(od))
    ref = orc.extend_attention(odesc(desc), host, 0, widen(q), qip, batch.block_indptr, batch.block_ids, ctx)
    assert_attention_close(oh, ref, dt)


def test_prep_host_equals_device_form():
    import torch

    L, Hq, Hkv, D, dt = SHAPES["qwen7b-bf16"]
    n = 33
    desc = PoolDesc(L, Hkv, Hq, D, 12, dt)
    host = normal(50, desc.shape, dt)
    qg = normal(51, (n, Hq, 2, D), dt)
    k, v = normal(52, (n, Hkv, D), dt), normal(53, (n, Hkv, D), dt)
    pos = np.random.default_rng(54).integers(0, 9000, n).astype(np.int32)
    slots = np.random.default_rng(55).choice(12 * 16, n, replace=False).astype(np.int32)
    wq = torch.from_numpy(np.random.default_rng(56).standard_normal(D).astype(np.float32)).cuda()
    wk = torch.from_numpy(np.random.default_rng(57).standard_normal(D).astype(np.float32)).cuda()
    inv = torch.from_numpy(dp.rope_inv_freq(D, 1e6)).cuda()
    res = []
    for hostform in (False, True):
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            p_ = pos if hostform else _i32(pos)
            s_ = slots.astype(np.uint32) if hostform else _i32(slots)
            o = pool.qk_norm_rope_append(1, to_device(qg), to_device(k), to_device(v), p_, s_, wq, wk, inv)
            pool.check()
            res.append((to_host(o), pool.read()))
    assert np.array_equal(bits(res[0][0]), bits(res[1][0]))
    assert np.array_equal(bits(res[0][1]), bits(res[1][1]))


def test_prep_host_reuses_equal_metadata_and_follows_changed_ones():
    """Every layer of a step passes the same positions and slots to the fused
    prep: the library uploads them once. Positions changed in place, slots
    changed in place and staging slots claimed by other host calls in
    between all get a fresh upload. Every call's output and the pool after
    all of them are bit-identical to the device-array form of the same
    calls."""
    import torch

    L, Hq, Hkv, D, dt = 3, 28, 4, 128, "bf16"
    n = 21
    desc = PoolDesc(L, Hkv, Hq, D, 16, dt)
    host = normal(90, desc.shape, dt)
    rng = np.random.default_rng(91)
    pos = rng.integers(0, 9000, n).astype(np.int32)
    slots = rng.choice(12 * 16, n, replace=False).astype(np.uint32)
    wq = torch.from_numpy(rng.standard_normal(D).astype(np.float32)).cuda()
    wk = torch.from_numpy(rng.standard_normal(D).astype(np.float32)).cuda()
    inv = torch.from_numpy(dp.rope_inv_freq(D, 1e6)).cuda()
    calls = []  # (layer, seed, positions, slots) as each call saw them

    def run(pool, hostform, layer, seed, p_, s_):
        qg = normal(seed, (n, Hq, 2, D), dt)
        k, v = normal(seed + 1, (n, Hkv, D), dt), normal(seed + 2, (n, Hkv, D), dt)
        a, b = (p_, s_) if hostform else (_i32(p_), _i32(s_))
        return to_host(pool.qk_norm_rope_append(layer, to_device(qg), to_device(k), to_device(v), a, b, wq, wk,
                                                inv))

    res = {}
    for hostform in (True, False):
        outs = []
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            if hostform:
                p_, s_ = pos.copy(), slots.copy()
                outs.append(run(pool, True, 0, 92, p_, s_))
                calls.append((0, 92, p_.copy(), s_.copy()))
                outs.append(run(pool, True, 1, 95, p_, s_))       # equal arrays: the staged copy
                calls.append((1, 95, p_.copy(), s_.copy()))
                p_ += 7                                           # positions changed in place
                outs.append(run(pool, True, 2, 98, p_, s_))
                calls.append((2, 98, p_.copy(), s_.copy()))
                s_[:] = rng.choice(np.setdiff1d(np.arange(12 * 16, 16 * 16), s_), n, replace=False)
                outs.append(run(pool, True, 0, 101, p_, s_))      # slots changed in place
                calls.append((0, 101, p_.copy(), s_.copy()))
                for i in range(9):                                # other host calls claim every staging slot
                    pool.copy_blocks(np.array([15], np.uint32), np.array([14 - i % 2], np.uint32))
                outs.append(run(pool, True, 1, 104, p_, s_))      # equal values, slot reused: uploaded again
                calls.append((1, 104, p_.copy(), s_.copy()))
            else:
                for i, (layer, seed, p_, s_) in enumerate(calls):
                    outs.append(run(pool, False, layer, seed, p_, s_))
                    if i == 3:
                        for j in range(9):
                            pool.copy_blocks(_i32([15]), _i32([14 - j % 2]))
            pool.check()
            res[hostform] = (outs, pool.read())
    for a, b in zip(res[True][0], res[False][0]):
        assert np.array_equal(bits(a), bits(b))
    assert np.array_equal(bits(res[True][1]), bits(res[False][1]))


def test_wire_host_equals_device_form_and_rejects_repeated_destinations():
    desc = PoolDesc(3, 4, 28, 128, 20, "bf16")
    host = normal(60, desc.shape, "bf16")
    ids = np.array([3, 0, 19, 7], np.int32)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        ph, ch = pool.wire_export(ids.astype(np.uint32))
        pd_, cd = pool.wire_export(_i32(ids))
        pool.check()
        assert np.array_equal(to_host(ph), to_host(pd_))
        assert np.array_equal(to_host(ch), to_host(cd))
        dst = np.array([10, 11, 12, 13], np.uint32)
        pool.wire_import(dst, ph, expected=ch)
        pool.check()
        after = pool.read()
        with pytest.raises(BackendError) as ei:
            pool.wire_import(np.array([5, 6, 5, 8], np.uint32), ph)
        assert "repeats" in str(ei.value)
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(after))
    want = host.copy()
    want[:, :, dst.astype(np.int64)] = host[:, :, ids]
    assert np.array_equal(bits(after), bits(want))


def test_append_host_reuses_an_equal_mapping_and_follows_a_changed_one():
    """Every layer of a step appends the same tokens: the library uploads an
    equal mapping once. A mapping changed in place under the same array, a
    staging slot claimed by other host calls in between, and another stream
    all get a fresh upload; every append is bit-exact."""
    import torch

    desc, pool, host = _pool("qwen7b-bf16", 64, 70)
    want = host.copy()
    rng = np.random.default_rng(71)
    slots = rng.choice(desc.num_blocks * 16, size=40, replace=False).astype(np.uint32)
    side = torch.cuda.Stream()

    def app(layer, seed, stream=None):
        k = normal(seed, (slots.size, desc.num_kv_heads, desc.head_dim), desc.dtype)
        v = normal(seed + 1, (slots.size, desc.num_kv_heads, desc.head_dim), desc.dtype)
        pool.append(layer, to_device(k), to_device(v), slots, stream=stream)
        orc.append(odesc(desc), want, layer, k, v, slots.astype(np.int32))

    app(0, 72)
    app(1, 74)                      # same mapping: launched from the staged copy
    slots[:] = rng.choice(desc.num_blocks * 16, size=40, replace=False)
    app(0, 76)                      # changed in place: uploaded again
    for i in range(9):              # other host calls claim every staging slot
        pool.copy_blocks(np.array([60], np.uint32), np.array([61 + i % 3], np.uint32))
        orc.copy_blocks(odesc(desc), want, np.array([60], np.int32), np.array([61 + i % 3], np.int32))
    app(1, 78)                      # equal values, but its slot was reused: uploaded again
    torch.cuda.synchronize()
    app(0, 80, stream=side)         # another stream: uploaded on it
    side.synchronize()
    pool.check()
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


def test_gather_host_reuses_equal_tables_and_follows_changed_ones():
    """Every layer of a step gathers the same tables: the library uploads
    equal tables once. Tables changed in place under the same arrays, new
    context lengths, staging slots claimed by other host calls in between,
    and another stream all get a fresh upload; every gather is bit-exact."""
    import torch

    rng = wl.SplitMix64(90)
    batch = wl.decode_batch_from_contexts([40, 300, 16, 7], rng, extra_blocks=12)
    desc, pool, host = _pool("qwen7b-bf16", batch.num_blocks, 91)
    ip = batch.block_indptr.astype(np.uint32)
    ids = batch.block_ids.astype(np.uint32)
    ctx = batch.ctx_lens.copy()
    side = torch.cuda.Stream()

    def check(layer, stream=None):
        kh, vh = pool.gather_host(layer, ip, ids, ctx, stream=stream)
        if stream is not None:
            stream.synchronize()
        wk, wv = orc.gather(odesc(desc), host, layer, ip.astype(np.int32), ids.astype(np.int32), ctx)
        assert np.array_equal(bits(to_host(kh)), bits(wk))
        assert np.array_equal(bits(to_host(vh)), bits(wv))

    check(0)
    check(1)                                  # equal tables: gathered from the staged copy
    free = np.setdiff1d(np.arange(desc.num_blocks), ids)
    ids[:3] = free[:3]                        # changed in place: uploaded again
    check(1)
    ctx[1] -= 17                              # shorter context, same tables
    check(0)
    for i in range(9):                        # other host calls claim every staging slot
        src, dst = np.array([free[5]], np.uint32), np.array([free[6 + i % 3]], np.uint32)
        pool.copy_blocks(src, dst)
        orc.copy_blocks(odesc(desc), host, src.astype(np.int32), dst.astype(np.int32))
    check(1)                                  # equal values, slot reused: uploaded again
    torch.cuda.synchronize()
    check(0, stream=side)                     # another stream: uploaded on it
    pool.check()
    pool.close()


def test_extend_host_reuses_equal_tables_and_follows_changed_ones():
    """Every layer of a chunked-prefill step passes the same chunks and
    tables: uploaded once, and re-uploaded when they change in place."""
    L, Hq, Hkv, D, dt = SHAPES["qwen7b-bf16"]
    rng = wl.SplitMix64(92)
    ctx = np.array([70, 300, 33], np.int32)
    ql = np.array([20, 64, 33], np.int32)
    batch = wl.decode_batch_from_contexts(list(ctx - 1), rng, extra_blocks=8)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    host = normal(93, desc.shape, dt)
    q = normal(94, (int(ql.sum()), Hq, D), dt)
    qip = np.zeros(ctx.size + 1, np.int32)
    np.cumsum(ql, out=qip[1:])
    ip = batch.block_indptr.astype(np.uint32)
    ids = batch.block_ids.astype(np.uint32)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        qd = to_device(q)

        def check(layer):
            got = to_host(pool.extend_attention_host(layer, qd, ql, ctx, ip, ids))
            ref = orc.extend_attention(odesc(desc), host, layer, widen(q), qip, ip.astype(np.int32),
                                       ids.astype(np.int32), ctx)
            assert_attention_close(got, ref, dt)
            return got

        a = check(0)
        b = check(0)                          # equal tables: launched from the staged copy
        assert np.array_equal(bits(a), bits(b))
        check(1)
        free = np.setdiff1d(np.arange(desc.num_blocks), ids)
        ids[-4:] = free[:4]                   # changed in place: uploaded again
        check(1)
        pool.check()
