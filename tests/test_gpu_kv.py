"""GPU parity: append / gather / copy_blocks bit-exact against the oracle, and
decode attention within the north-star tolerances (f32 max-abs 1e-5, bf16
row-relative 2e-2), all through the C ABI of libmitten_kv."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import BackendError, DeviceIndexError, DeviceKvPool, PoolDesc
from mitten_amd import device_pool as dp
from mitten_amd import workloads as wl
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

SHAPES = {
    # name: (layers, Hq, Hkv, D, dtype)
    "qwen0.5b-f32": (3, 14, 2, 64, "f32"),
    "qwen7b-bf16": (2, 28, 4, 128, "bf16"),
    "gemma2b-bf16": (2, 8, 1, 256, "bf16"),
    "qwen0.5b-bf16": (2, 14, 2, 64, "bf16"),
    "llama8b-bf16": (1, 32, 8, 128, "bf16"),
    "g16-bf16": (1, 64, 4, 128, "bf16"),
    "d256-g4-bf16": (1, 16, 4, 256, "bf16"),  # head_dim 256, 2 Q loads per lane in the cooperative kernel
    "d256-g2-bf16": (1, 4, 2, 256, "bf16"),   # head_dim 256, 1 Q load per lane
    "d32-f32": (1, 12, 2, 32, "f32"),         # the per-head kernel's other head dims, f32
    "d128-f32": (1, 14, 2, 128, "f32"),
    "d256-f32": (1, 8, 1, 256, "f32"),
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
def test_append_bit_exact(shape):
    desc, pool, host = _pool(shape, 40, 1)
    rng = np.random.default_rng(2)
    n = 37
    slots = rng.choice(desc.num_blocks * 16, size=n, replace=False).astype(np.int32)
    k = normal(3, (n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(4, (n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    layer = desc.num_layers - 1
    pool.append(layer, to_device(k), to_device(v), _i32(slots))
    pool.check()
    got = pool.read()
    want = host.copy()
    assert orc.append(odesc(desc), want, layer, k, v, slots) == -1
    assert np.array_equal(bits(got), bits(want))
    pool.close()


@pytest.mark.parametrize("shape", ["qwen0.5b-f32", "qwen7b-bf16"])
def test_append_all_layers_bit_exact(shape):
    desc, pool, host = _pool(shape, 24, 5)
    n = 50
    slots = np.random.default_rng(6).choice(desc.num_blocks * 16, size=n, replace=False).astype(np.int32)
    k = normal(7, (desc.num_layers, n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(8, (desc.num_layers, n, desc.num_kv_heads, desc.head_dim), desc.dtype)
    pool.append_all_layers(to_device(k), to_device(v), _i32(slots))
    pool.check()
    want = host.copy()
    for layer in range(desc.num_layers):
        orc.append(odesc(desc), want, layer, np.ascontiguousarray(k[layer]), np.ascontiguousarray(v[layer]), slots)
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


def test_append_out_of_range_slot_is_reported_and_skipped():
    desc, pool, host = _pool("qwen7b-bf16", 8, 9)
    slots = np.array([3, desc.num_blocks * 16, -1, 17], np.int32)
    k = normal(10, (4, desc.num_kv_heads, desc.head_dim), desc.dtype)
    v = normal(11, (4, desc.num_kv_heads, desc.head_dim), desc.dtype)
    pool.append(0, to_device(k), to_device(v), _i32(slots))
    with pytest.raises(DeviceIndexError) as ei:
        pool.check()
    assert ei.value.bits & dp.DEVERR_SLOT
    want = host.copy()
    good = np.array([0, 3])
    orc.append(odesc(desc), want, 0, np.ascontiguousarray(k[good]), np.ascontiguousarray(v[good]), slots[good])
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.check()  # the error word was cleared
    pool.close()


@pytest.mark.parametrize("shape", list(SHAPES))
def test_gather_bit_exact(shape):
    rng = wl.SplitMix64(12)
    ctx = [1, 15, 16, 17, 100, 333]
    batch = wl.decode_batch_from_contexts(ctx, rng, extra_blocks=5)
    desc, pool, host = _pool(shape, batch.num_blocks, 13)
    layer = desc.num_layers - 1
    ci = batch.ctx_indptr
    k, v = pool.gather(layer, _i32(batch.block_indptr), _i32(batch.block_ids), _i32(ci), batch.max_ctx,
                       total_tokens=int(ci[-1]))
    pool.check()
    wk, wv = orc.gather(odesc(desc), host, layer, batch.block_indptr, batch.block_ids, batch.ctx_lens)
    assert np.array_equal(bits(to_host(k)), bits(wk))
    assert np.array_equal(bits(to_host(v)), bits(wv))
    pool.close()


def test_append_then_gather_equals_contiguous_cat():
    """Appending tokens one at a time and gathering yields the contiguous
    cache Tensor::cat builds (model.rs:390-392), in [heads, seq, dim] order."""
    import torch

    desc = PoolDesc(1, 2, 14, 64, 12, "f32")
    with DeviceKvPool(desc) as pool:
        pool.write(normal(14, desc.shape, "f32"))
        rng = wl.SplitMix64(15)
        table = wl.permutation(desc.num_blocks, rng)[:9]
        n = 131
        ks = normal(16, (n, 2, 64), "f32")
        vs = normal(17, (n, 2, 64), "f32")
        for t in range(n):
            slot = np.array([table[t // 16] * 16 + t % 16], np.int32)
            pool.append(0, to_device(ks[t:t + 1]), to_device(vs[t:t + 1]), _i32(slot))
        k, v = pool.gather(0, _i32([0, 9]), _i32(table), _i32([0, n]), n, total_tokens=n)
        pool.check()
        assert np.array_equal(to_host(k).reshape(2, n, 64), ks.transpose(1, 0, 2))
        assert np.array_equal(to_host(v).reshape(2, n, 64), vs.transpose(1, 0, 2))
        torch.cuda.synchronize()


@pytest.mark.parametrize("shape", list(SHAPES))
def test_copy_blocks_bit_exact(shape):
    desc, pool, host = _pool(shape, 64, 18)
    rng = np.random.default_rng(19)
    ids = rng.permutation(desc.num_blocks).astype(np.int32)
    src, dst = ids[:20], ids[20:40]
    dp.validate_copy_pairs(desc, src, dst)
    pool.copy_blocks(_i32(src), _i32(dst))
    pool.check()
    want = host.copy()
    orc.copy_blocks(odesc(desc), want, src, dst)
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


def test_copy_blocks_bad_id_reported():
    desc, pool, host = _pool("qwen7b-bf16", 8, 20)
    pool.copy_blocks(_i32([1, 2]), _i32([5, 99]))
    with pytest.raises(DeviceIndexError) as ei:
        pool.check()
    assert ei.value.bits & dp.DEVERR_COPY
    want = host.copy()
    orc.copy_blocks(odesc(desc), want, [1], [5])
    assert np.array_equal(bits(pool.read()), bits(want))
    pool.close()


# ---------------------------------------------------------------- attention ----

def _attention_case(shape, ctx, seed, kernel=None, split_tokens=0, zero_sink=False, layer=None):
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(seed)
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng, extra_blocks=3)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    layer = L - 1 if layer is None else layer
    with DeviceKvPool(desc) as pool:
        host = normal(seed + 1, desc.shape, dt)
        pool.write(host)
        q = normal(seed + 2, (len(ctx), Hq, D), dt)
        o = pool.decode_attention(layer, to_device(q), _i32(batch.block_indptr), _i32(batch.block_ids),
                                  _i32(batch.ctx_lens), batch.max_ctx, zero_sink=zero_sink,
                                  split_tokens=split_tokens, kernel=kernel)
        pool.check()
        got = to_host(o)
    ref = orc.decode_attention(odesc(desc), host, layer, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens, zero_sink=zero_sink)
    return got, ref, dt


CTX_EDGE = [1, 2, 15, 16, 17, 31, 32, 33, 127, 128, 129, 257, 500, 1000]


@pytest.mark.parametrize("split_tokens", [0, 16, 48, 128])
def test_attention_f32_gqa(split_tokens):
    got, ref, dt = _attention_case("qwen0.5b-f32", CTX_EDGE, 30, split_tokens=split_tokens)
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
@pytest.mark.parametrize("split_tokens", [0, 32, 256])
def test_attention_bf16_gqa(kernel, split_tokens):
    got, ref, dt = _attention_case("qwen7b-bf16", CTX_EDGE, 31, kernel=kernel, split_tokens=split_tokens)
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
def test_attention_bf16_mqa_wide_head(kernel):
    got, ref, dt = _attention_case("gemma2b-bf16", CTX_EDGE, 32, kernel=kernel)
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("shape,kernel", [("qwen0.5b-f32", None), ("qwen7b-bf16", "mfma"),
                                          ("qwen7b-bf16", "valu")])
def test_attention_zero_sink(shape, kernel):
    got, ref, dt = _attention_case(shape, [1, 5, 40, 300], 33, kernel=kernel, zero_sink=True, split_tokens=32)
    assert_attention_close(got, ref, dt)


def test_attention_bad_block_id_reported():
    desc = PoolDesc(1, 4, 28, 128, 10, "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(normal(40, desc.shape, "bf16"))
        q = to_device(normal(41, (2, 28, 128), "bf16"))
        pool.decode_attention(0, q, _i32([0, 2, 4]), _i32([1, 2, 3, 10]), _i32([20, 30]), 30)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_BLOCK


def test_attention_short_table_reported():
    desc = PoolDesc(1, 4, 28, 128, 10, "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(normal(42, desc.shape, "bf16"))
        q = to_device(normal(43, (1, 28, 128), "bf16"))
        pool.decode_attention(0, q, _i32([0, 1]), _i32([4]), _i32([40]), 40)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_TABLE


@pytest.mark.parametrize("name", ["qwen2.5-7b", "gemma-2b-mqa"])
def test_attention_full_config_one_layer(name):
    """One layer at the configuration's full batch and context lengths."""
    c = wl.CONFIGS[name]
    batch = wl.config_batch(name)
    desc = PoolDesc(1, c["num_kv_heads"], c["num_q_heads"], c["head_dim"], batch.num_blocks, c["dtype"])
    with DeviceKvPool(desc) as pool:
        host = normal(50, desc.shape, desc.dtype)
        pool.write(host)
        q = normal(51, (batch.num_seqs, desc.num_q_heads, desc.head_dim), desc.dtype)
        o = pool.decode_attention(0, to_device(q), _i32(batch.block_indptr), _i32(batch.block_ids),
                                  _i32(batch.ctx_lens), batch.max_ctx)
        pool.check()
        got = to_host(o)
    ref = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens)
    assert_attention_close(got, ref, desc.dtype)


# ------------------------------------------------------------ planned path ----

def _planned_case(shape, ctx, seed, pieces=0, kernel=None, zero_sink=False, fused=False):
    """Returns (got, ref, dtype, pool_after, pool_want) for one layer."""
    L, Hq, Hkv, D, dt = SHAPES[shape]
    rng = wl.SplitMix64(seed)
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng, extra_blocks=3)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    layer = L - 1
    B = len(ctx)
    host = normal(seed + 1, desc.shape, dt)
    q = normal(seed + 2, (B, Hq, D), dt)
    kn = normal(seed + 3, (B, Hkv, D), dt)
    vn = normal(seed + 4, (B, Hkv, D), dt)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan(batch.ctx_lens, pieces=pieces)
        args = (_i32(batch.block_indptr), _i32(batch.block_ids))
        if fused:
            o = pool.decode_step(layer, plan, to_device(kn), to_device(vn), to_device(q), *args,
                                 zero_sink=zero_sink, kernel=kernel)
        else:
            o = pool.decode_attention_planned(layer, plan, to_device(q), *args, zero_sink=zero_sink, kernel=kernel)
        pool.check()
        got = to_host(o)
        after = pool.read()
        info = plan.info()
        plan.close()
    want = host.copy()
    if fused:
        assert orc.append(odesc(desc), want, layer, kn, vn, batch.slot_mapping) == -1
    ref = orc.decode_attention(odesc(desc), want, layer, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens, zero_sink=zero_sink)
    return got, ref, dt, after, want, info


PLAN_CTX = [1, 2, 15, 16, 17, 33, 100, 129, 257, 500, 1000, 3, 64, 65, 700]


# Planned-path kernels: "mfma" takes the cooperative whole-row loader where
# the workgroup holds every KV head (Hkv <= 4, G <= 16) and the per-head
# stream kernel otherwise (llama8b: Hkv = 8); "mfma-per-head" forces the latter.
PLANNED_KERNELS = [("qwen0.5b-f32", None), ("qwen7b-bf16", "mfma"), ("qwen7b-bf16", "mfma-per-head"),
                   ("qwen7b-bf16", "valu"), ("gemma2b-bf16", "mfma"), ("gemma2b-bf16", "mfma-per-head"),
                   ("qwen0.5b-bf16", "mfma"), ("llama8b-bf16", "mfma"), ("g16-bf16", "mfma"),
                   ("d256-g4-bf16", "mfma"), ("d256-g2-bf16", "mfma"), ("d256-g4-bf16", "mfma-per-head")]


@pytest.mark.parametrize("pieces", [0, 1, 7, 40, 300])
@pytest.mark.parametrize("shape,kernel", PLANNED_KERNELS)
def test_planned_attention(shape, kernel, pieces):
    got, ref, dt, after, want, info = _planned_case(shape, PLAN_CTX, 60, pieces=pieces, kernel=kernel)
    assert_attention_close(got, ref, dt)
    assert np.array_equal(bits(after), bits(want))  # attention never writes the pool


@pytest.mark.parametrize("pieces", [0, 5, 64])
@pytest.mark.parametrize("shape,kernel", PLANNED_KERNELS)
def test_decode_step_fused_append(shape, kernel, pieces):
    got, ref, dt, after, want, info = _planned_case(shape, PLAN_CTX, 61, pieces=pieces, kernel=kernel, fused=True)
    assert np.array_equal(bits(after), bits(want)), "fused append is not bit-exact"
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("ctx", [PLAN_CTX, [480 + 7 * i for i in range(40)]])
@pytest.mark.parametrize("shape,kernel", [("qwen0.5b-f32", None), ("qwen0.5b-bf16", "valu")])
def test_per_head_kernel_small_and_wide_query_chunks(shape, kernel, ctx):
    """The per-head kernel takes 1 query head per wave for a launch with
    fewer (block, KV head) units than two per CU (PLAN_CTX: 191 blocks x 2
    heads) and 8 per wave otherwise (40 sequences of ~600 tokens: ~1,500 x 2).
    Both, with G = 7 (seven chunks of 1, and one of 7), fused append
    included, against the oracle."""
    got, ref, dt, after, want, info = _planned_case(shape, ctx, 62, kernel=kernel, fused=True)
    assert np.array_equal(bits(after), bits(want)), "fused append is not bit-exact"
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("small", [True, False])
@pytest.mark.parametrize("shape,kernel", [("d32-f32", None), ("d128-f32", None), ("d256-f32", None),
                                          ("qwen7b-bf16", "valu"), ("gemma2b-bf16", "valu"), ("g16-bf16", "valu")])
def test_per_head_kernel_query_chunks_every_head_dim(shape, kernel, small):
    """Both query-chunk widths of the per-head kernel at head_dim 32, 128 and
    256 (f32, and bf16 forced onto it): a few short sequences (under two
    (block, KV head) units per CU: 1 head per wave) and forty of ~600 tokens
    (8 per wave), fused append included, against the oracle."""
    ctx = [1, 17, 40, 100, 33] if small else [480 + 7 * i for i in range(40)]
    got, ref, dt, after, want, info = _planned_case(shape, ctx, 63, kernel=kernel, fused=True)
    assert np.array_equal(bits(after), bits(want)), "fused append is not bit-exact"
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("kernel", ["mfma", "mfma-per-head", "valu"])
def test_planned_bad_block_id_reported(kernel):
    """An id outside the pool is reported and its block skipped; the other
    sequence of the batch is unaffected and nothing is written for it."""
    desc = PoolDesc(1, 4, 28, 128, 10, "bf16")
    host = normal(80, desc.shape, "bf16")
    q = normal(81, (2, 28, 128), "bf16")
    kn, vn = normal(82, (2, 4, 128), "bf16"), normal(83, (2, 4, 128), "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan([20, 30])
        o = pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), _i32([0, 2, 4]),
                             _i32([1, 2, 3, 10]), kernel=kernel)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_BLOCK
        got = to_host(o)
        after = pool.read()
        plan.close()
    want = host.copy()
    assert orc.append(odesc(desc), want, 0, kn[:1], vn[:1], np.array([2 * 16 + 3], np.int32)) == -1
    assert np.array_equal(bits(after), bits(want))
    ref = orc.decode_attention(odesc(desc), want, 0, widen(q[:1]), np.array([0, 2], np.int32),
                               np.array([1, 2], np.int32), np.array([20], np.int32))
    assert_attention_close(got[:1], ref, "bf16")


@pytest.mark.parametrize("shape", ["qwen0.5b-f32", "qwen7b-bf16"])
def test_planned_zero_sink(shape):
    got, ref, dt, *_ = _planned_case(shape, [1, 7, 40, 300], 62, pieces=9, zero_sink=True, fused=True)
    assert_attention_close(got, ref, dt)


@pytest.mark.parametrize("shape", ["qwen7b-bf16", "gemma2b-bf16"])
def test_cached_loads_on_shared_prefix_tables(shape):
    """Tables that share a prefix's blocks (as after radix sharing), decoded
    with the cache-resident loads (MKV_ATTN_CACHED_LOADS): the fused step
    appends bit-exactly, the outputs are bit-identical to the non-temporal
    default and match the oracle."""
    L, Hq, Hkv, D, dt = SHAPES[shape]
    batch = wl.shared_prefix_batch(24, 300, 5, 90, wl.SplitMix64(66))
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    host = normal(67, desc.shape, dt)
    B = batch.num_seqs
    q = normal(68, (B, Hq, D), dt)
    kn, vn = normal(69, (B, Hkv, D), dt), normal(70, (B, Hkv, D), dt)
    outs = []
    for cached in (False, True):
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            plan = pool.plan(batch.ctx_lens, pieces=11)
            o = pool.decode_step(L - 1, plan, to_device(kn), to_device(vn), to_device(q), _i32(batch.block_indptr),
                                 _i32(batch.block_ids), kernel="mfma", cached_loads=cached)
            pool.check()
            outs.append((to_host(o), pool.read()))
            plan.close()
    want = host.copy()
    assert orc.append(odesc(desc), want, L - 1, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(outs[1][1]), bits(want))
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))
    ref = orc.decode_attention(odesc(desc), want, L - 1, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens)
    assert_attention_close(outs[1][0], ref, dt)


@pytest.mark.parametrize("name", ["qwen2.5-7b", "gemma-2b-mqa"])
def test_decode_step_full_config_one_layer(name):
    """Fused append + planned attention at the configuration's full size."""
    c = wl.CONFIGS[name]
    batch = wl.config_batch(name)
    desc = PoolDesc(1, c["num_kv_heads"], c["num_q_heads"], c["head_dim"], batch.num_blocks, c["dtype"])
    B = batch.num_seqs
    host = normal(70, desc.shape, desc.dtype)
    q = normal(71, (B, desc.num_q_heads, desc.head_dim), desc.dtype)
    kn = normal(72, (B, desc.num_kv_heads, desc.head_dim), desc.dtype)
    vn = normal(73, (B, desc.num_kv_heads, desc.head_dim), desc.dtype)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan(batch.ctx_lens)
        o = pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), _i32(batch.block_indptr),
                             _i32(batch.block_ids))
        pool.check()
        got = to_host(o)
        after = pool.read()
        plan.close()
    assert orc.append(odesc(desc), host, 0, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(after), bits(host))
    ref = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens)
    assert_attention_close(got, ref, desc.dtype)


def test_bound_decode_step_matches_per_call():
    """bind_decode_step (validated once, bare ABI calls per layer) gives the
    same pool and outputs as decode_step called layer by layer."""
    import torch

    L, Hq, Hkv, D, dt = SHAPES["qwen7b-bf16"]
    rng = wl.SplitMix64(80)
    batch = wl.decode_batch_from_contexts([30, 200, 1, 77], rng, extra_blocks=2)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    host = normal(81, desc.shape, dt)
    B = batch.num_seqs
    q = to_device(normal(82, (L, B, Hq, D), dt))
    kn = to_device(normal(83, (L, B, Hkv, D), dt))
    vn = to_device(normal(84, (L, B, Hkv, D), dt))
    ip, ix = _i32(batch.block_indptr), _i32(batch.block_ids)
    results = []
    for bound in (False, True):
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            plan = pool.plan(batch.ctx_lens, pieces=3)
            out = torch.empty_like(q)
            run = pool.bind_decode_step(plan, kn, vn, q, ip, ix, out) if bound else None
            for layer in range(L):
                if bound:
                    run(layer)
                else:
                    pool.decode_step(layer, plan, kn[layer], vn[layer], q[layer], ip, ix, out=out[layer])
            pool.check()
            results.append((pool.read(), to_host(out)))
            plan.close()
    assert np.array_equal(bits(results[0][0]), bits(results[1][0]))
    assert np.array_equal(bits(results[0][1]), bits(results[1][1]))


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
def test_launch_events_bracket_the_next_attention_kernel_once(kernel):
    """The measurement hook records its two events around the next decode
    call's attention kernel only (one shot); the results are unchanged."""
    import torch

    desc = PoolDesc(1, 4, 28, 128, 40, "bf16") if kernel == "mfma" else PoolDesc(1, 2, 14, 64, 40, "f32")
    dt = desc.dtype
    host = normal(84, desc.shape, dt)
    q = normal(85, (3, desc.num_q_heads, desc.head_dim), dt)
    kn, vn = (normal(s, (3, desc.num_kv_heads, desc.head_dim), dt) for s in (86, 87))
    ip, ids = _i32([0, 3, 5, 12]), _i32(np.arange(12) + 20)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan([40, 20, 100])
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        b.record()  # torch creates its events at their first record
        torch.cuda.synchronize()
        pool.set_launch_events(a, b)
        o1 = to_host(pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), ip, ids, kernel=kernel))
        torch.cuda.synchronize()
        first = a.elapsed_time(b)
        assert first > 0.0
        o2 = to_host(pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), ip, ids, kernel=kernel))
        torch.cuda.synchronize()
        assert a.elapsed_time(b) == first  # not recorded again
        with pytest.raises(BackendError):
            pool.set_launch_events(a, None)
        pool.set_launch_events(None, None)
        pool.check()
        plan.close()
    assert np.array_equal(bits(o1), bits(o2))


@pytest.mark.parametrize("held", [False, True])
@pytest.mark.parametrize("pieces", [0, 1, 7, 300])
@pytest.mark.parametrize("shape,kernel", [("qwen0.5b-f32", None), ("qwen7b-bf16", "valu"),
                                          ("qwen7b-bf16", "mfma"), ("gemma2b-bf16", "mfma-per-head")])
def test_decode_step_gather_equals_step_then_gather(shape, kernel, pieces, held):
    """The step with its gather (stored by the per-head kernel as it reads
    the rows, or the gather kernel after the MFMA kernels) is bit-identical
    to mkv_decode_step followed by mkv_gather: output, pool and both gathered
    caches, which equal the oracle's gather of the appended pool. held: the
    plan holds the host tables and the calls pass none."""
    import torch

    L, Hq, Hkv, D, dt = SHAPES[shape]
    ctx = [1, 2, 15, 16, 17, 33, 100, 257, 500, 64]
    rng = wl.SplitMix64(63)
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng, extra_blocks=3)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    layer = L - 1
    B = len(ctx)
    host = normal(64, desc.shape, dt)
    q = normal(65, (B, Hq, D), dt)
    kn, vn = normal(66, (B, Hkv, D), dt), normal(67, (B, Hkv, D), dt)
    ntok = int(sum(ctx)) * Hkv * D
    res = []
    for with_gather in (True, False):
        with DeviceKvPool(desc) as pool:
            pool.write(host)
            dev_tables = (_i32(batch.block_indptr), _i32(batch.block_ids))
            if held:
                plan = pool.plan(batch.ctx_lens, pieces=pieces, block_indptr=batch.block_indptr.astype(np.uint32),
                                 block_ids=batch.block_ids.astype(np.uint32))
                args = (None, None)
            else:
                plan = pool.plan(batch.ctx_lens, pieces=pieces)
                args = dev_tables
            if with_gather:
                gk = torch.full((ntok + 8,), 7.0, dtype=pool.torch_dtype, device="cuda")
                gv = torch.full_like(gk, 7.0)
                o = pool.decode_step(layer, plan, to_device(kn), to_device(vn), to_device(q), *args, kernel=kernel,
                                     gather_out=(gk, gv))
                gk, gv = to_host(gk[:ntok]), to_host(gv[:ntok])
            else:
                o = pool.decode_step(layer, plan, to_device(kn), to_device(vn), to_device(q), *args, kernel=kernel)
                gk, gv = (to_host(t) for t in pool.gather(layer, *dev_tables, _i32(batch.ctx_indptr), batch.max_ctx))
            pool.check()
            res.append((to_host(o), pool.read(), gk, gv))
            plan.close()
    (o1, p1, k1, v1), (o2, p2, k2, v2) = res
    assert np.array_equal(bits(o1), bits(o2))
    assert np.array_equal(bits(p1), bits(p2))
    assert np.array_equal(bits(k1), bits(k2)) and np.array_equal(bits(v1), bits(v2))
    want = host.copy()
    assert orc.append(odesc(desc), want, layer, kn, vn, batch.slot_mapping) == -1
    wk, wv = orc.gather(odesc(desc), want, layer, batch.block_indptr, batch.block_ids, batch.ctx_lens)
    assert np.array_equal(bits(k1), bits(wk)) and np.array_equal(bits(v1), bits(wv))


def test_decode_step_gather_rejects_small_outputs():
    import torch

    desc = PoolDesc(1, 2, 14, 64, 8, "f32")
    with DeviceKvPool(desc) as pool:
        plan = pool.plan([20, 30])
        z = torch.zeros((2, 2, 64), dtype=torch.float32, device="cuda")
        q = torch.zeros((2, 14, 64), dtype=torch.float32, device="cuda")
        small = torch.zeros(49 * 2 * 64, dtype=torch.float32, device="cuda")  # 49 < 50 tokens
        with pytest.raises(BackendError):
            pool.decode_step(0, plan, z, z, q, _i32([0, 2, 4]), _i32([0, 1, 2, 3]), gather_out=(small, small))
        plan.close()


def test_device_buffers_and_pool_descriptor_through_the_abi():
    """The backend's device-buffer entry points (mkv_buffer_alloc / free,
    memcpy both ways) round-trip bytes; mkv_pool_get_desc returns the
    descriptor the pool was made from and mkv_pool_buffer its size; NULL
    outputs and a device that does not exist are refused with a status, and
    leave no HIP error for the caller's next check."""
    import ctypes

    from mitten_amd import _lib, required_bytes

    lib = _lib.device_lib()
    n = 3 * 4096 + 48
    src = np.random.default_rng(41).integers(0, 256, n, dtype=np.uint8)
    back = np.zeros(n, np.uint8)
    ptr = ctypes.c_void_p()
    assert lib.mkv_buffer_alloc(0, n, ctypes.byref(ptr)) == 0 and ptr.value
    try:
        assert lib.mkv_memcpy_h2d(ptr, src.ctypes.data_as(ctypes.c_void_p), n, None) == 0
        assert lib.mkv_memcpy_d2h(back.ctypes.data_as(ctypes.c_void_p), ptr, n, None) == 0
        assert np.array_equal(back, src)
    finally:
        assert lib.mkv_buffer_free(ptr) == 0
    assert lib.mkv_buffer_free(None) == 0
    assert lib.mkv_buffer_alloc(0, 16, None) == dp.MKV_ERR_INVALID_ARGUMENT
    bad = ctypes.c_void_p()
    assert lib.mkv_buffer_alloc(4096, 16, ctypes.byref(bad)) == dp.MKV_ERR_INVALID_ARGUMENT and not bad.value
    assert b"out of range" in lib.mkv_last_error()
    # A refused call leaves no HIP error behind for the caller's next check.
    import torch

    assert torch.zeros(4, device="cuda").sum().item() == 0.0

    desc = PoolDesc(3, 4, 28, 128, 37, "bf16")
    with DeviceKvPool(desc) as pool:
        got = _lib.PoolDescC()
        assert lib.mkv_pool_get_desc(pool._h, ctypes.byref(got)) == 0
        want = desc.c()
        assert [getattr(got, f) for f, _ in got._fields_] == [getattr(want, f) for f, _ in want._fields_]
        assert lib.mkv_pool_get_desc(pool._h, None) == dp.MKV_ERR_INVALID_ARGUMENT
        size = ctypes.c_uint64()
        base = ctypes.c_void_p()
        assert lib.mkv_pool_buffer(pool._h, ctypes.byref(base), ctypes.byref(size)) == 0
        assert size.value == required_bytes(desc) and base.value == pool.data_ptr


@pytest.mark.parametrize("ctx,pieces,zero_sink", [([4096], 0, False), ([4096], 0, True), ([700, 1900, 64], 0, False),
                                                  ([700, 1900, 64], 166, True), ([1024] * 4, 256, False)])
def test_rows_of_many_partials_merge_over_waves(ctx, pieces, zero_sink):
    """A small batch cut into many short pieces (the device's choice: pieces of
    4 blocks, at most one per CU; or an explicit count) leaves rows of more
    than 16 partials, which the merge spreads over 8 waves and combines in
    LDS. Fused step vs the oracle at Qwen2.5-7B heads."""
    import torch

    Hq, Hkv, D = 28, 4, 128
    seed = 71 + len(ctx) + pieces
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], wl.SplitMix64(seed), extra_blocks=2)
    desc = PoolDesc(1, Hkv, Hq, D, batch.num_blocks, "bf16")
    host = normal(seed + 1, desc.shape, "bf16")
    B = len(ctx)
    q = normal(seed + 2, (B, Hq, D), "bf16")
    kn, vn = normal(seed + 3, (B, Hkv, D), "bf16"), normal(seed + 4, (B, Hkv, D), "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan(batch.ctx_lens, pieces=pieces)
        info = plan.info()
        most = max(-(-c // 16) for c in ctx) / max(info["blocks_per_piece"], 1)
        assert most > 16, info  # some row has more partials than one round of the narrow merge
        o = pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), _i32(batch.block_indptr),
                             _i32(batch.block_ids), zero_sink=zero_sink)
        pool.check()
        got, after = to_host(o), pool.read()
        plan.close()
    want = host.copy()
    assert orc.append(odesc(desc), want, 0, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(after), bits(want))
    ref = orc.decode_attention(odesc(desc), want, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens,
                               zero_sink=zero_sink)
    assert_attention_close(got, ref, "bf16")
