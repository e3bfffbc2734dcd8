"""GPU parity of decode over a shared prefix (mkv_decode_step_shared_prefix)
through the C ABI: every sequence's tables start with the same full prefix
blocks (as radix sharing hands them out); the step reads the prefix once for
all sequences on MFMA tiles, the suffixes through the plan, and merges both.
Checked against the oracle's decode attention over the whole tables (bf16
row-relative 2e-2), with the fused append bit-exact, plus the error paths."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import BackendError, DeviceKvPool, PoolDesc
from mitten_amd import workloads as wl
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

SHAPES = {
    # name: (layers, Hq, Hkv, D)
    "qwen7b": (2, 28, 4, 128),
    "gemma2b": (1, 8, 1, 256),
    "qwen0.5b": (1, 14, 2, 64),
    "llama8b": (1, 32, 8, 128),  # suffixes on the per-head stream kernel
    "g16": (1, 64, 4, 128),
    "d256-g4": (1, 16, 4, 256),   # head_dim 256: 4-wave prefix workgroups, 4 KV heads per suffix workgroup
    "d256-g16": (1, 16, 1, 256),  # head_dim 256: 16-wave prefix workgroups, per-head suffix kernel
}


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _split_tables(batch, full):
    """Suffix tables (each table past its first `full` blocks) and lengths."""
    ip = batch.block_indptr
    tabs = [batch.block_ids[ip[b] + full:ip[b + 1]] for b in range(batch.num_seqs)]
    sptr = np.concatenate([[0], np.cumsum([len(t) for t in tabs])]).astype(np.int32)
    return sptr, np.concatenate(tabs).astype(np.int32), (batch.ctx_lens - 16 * full).astype(np.int32)


def _case(shape, seqs, prefix, lo, hi, seed, zero_sink=False, fused=True, pieces=0, repeats=1):
    L, Hq, Hkv, D = SHAPES[shape]
    batch = wl.shared_prefix_batch(seqs, prefix, lo, hi, wl.SplitMix64(seed))
    full = prefix // 16
    sptr, sids, slen = _split_tables(batch, full)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, "bf16")
    host = normal(seed + 1, desc.shape, "bf16")
    q = normal(seed + 2, (seqs, Hq, D), "bf16")
    kn, vn = normal(seed + 3, (seqs, Hkv, D), "bf16"), normal(seed + 4, (seqs, Hkv, D), "bf16")
    layer = L - 1
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan_suffixes(slen, pieces=pieces)
        outs = []
        for _ in range(repeats):
            o = pool.decode_step_shared_prefix(layer, plan, to_device(kn) if fused else None,
                                               to_device(vn) if fused else None, to_device(q),
                                               _i32(batch.meta["shared_blocks"]), _i32(sptr), _i32(sids),
                                               zero_sink=zero_sink)
            pool.check()
            outs.append(to_host(o))
        after = pool.read()
        plan.close()
    want = host.copy()
    if fused:
        assert orc.append(odesc(desc), want, layer, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(after), bits(want))
    ref = orc.decode_attention(odesc(desc), want, layer, widen(q), batch.block_indptr, batch.block_ids,
                               batch.ctx_lens, zero_sink=zero_sink)
    return outs, ref


@pytest.mark.parametrize("shape", list(SHAPES))
def test_shared_prefix_matches_oracle(shape):
    outs, ref = _case(shape, 24, 300, 1, 90, 120)
    assert_attention_close(outs[0], ref, "bf16")


@pytest.mark.parametrize("prefix,seqs,lo,hi", [
    (16, 5, 1, 3),        # one prefix block, suffixes of 1..3 tokens (the new token's block alone)
    (4100, 64, 64, 1024),  # the shared-prefix configuration's prefix: the prefix splits in 16 key ranges
    (64, 300, 1, 40),     # more sequences than one 256-query tile row
])
def test_shared_prefix_sizes(prefix, seqs, lo, hi):
    outs, ref = _case("qwen7b", seqs, prefix, lo, hi, 121)
    assert_attention_close(outs[0], ref, "bf16")


def test_shared_prefix_zero_sink_no_append_one_piece_and_repeats():
    outs, ref = _case("qwen7b", 12, 500, 10, 200, 122, zero_sink=True, fused=False, pieces=1, repeats=3)
    for o in outs:
        assert_attention_close(o, ref, "bf16")
    assert all(np.array_equal(bits(o), bits(outs[0])) for o in outs)


def test_shared_prefix_between_extend_calls():
    """The prefix partials share the pool workspace with split extend
    attention: calls of both on one stream, interleaved, stay correct."""
    L, Hq, Hkv, D = SHAPES["qwen7b"]
    batch = wl.shared_prefix_batch(16, 2000, 20, 300, wl.SplitMix64(123))
    full = 2000 // 16
    sptr, sids, slen = _split_tables(batch, full)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, "bf16")
    host = normal(124, desc.shape, "bf16")
    q = normal(125, (16, Hq, D), "bf16")
    qe = normal(126, (16 * 8, Hq, D), "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        plan = pool.plan_suffixes(slen)
        qi = _i32(np.arange(17) * 8)
        args = (_i32(batch.block_indptr), _i32(batch.block_ids), _i32(batch.ctx_lens))
        for _ in range(2):
            oe = pool.extend_attention(0, to_device(qe), qi, *args, 8, int(batch.ctx_lens.max()))
            o = pool.decode_step_shared_prefix(0, plan, None, None, to_device(q), _i32(batch.meta["shared_blocks"]),
                                               _i32(sptr), _i32(sids))
        pool.check()
        got, got_e = to_host(o), to_host(oe)
        plan.close()
    ref = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens)
    assert_attention_close(got, ref, "bf16")
    ref_e = orc.extend_attention(odesc(desc), host, 0, widen(qe), np.arange(17) * 8, batch.block_indptr,
                                 batch.block_ids, batch.ctx_lens)
    assert_attention_close(got_e, ref_e, "bf16")


def test_shared_prefix_errors():
    import torch

    desc = PoolDesc(1, 4, 28, 128, 12, "bf16")
    with DeviceKvPool(desc) as pool:
        q = torch.zeros((2, 28, 128), dtype=torch.bfloat16, device="cuda")
        plain = pool.plan([5, 9])
        with pytest.raises(BackendError):  # a plan not built over suffixes
            pool.decode_step_shared_prefix(0, plain, None, None, q, _i32([0, 1]), _i32([0, 1, 2]), _i32([2, 3]))
        plain.close()
        sp = pool.plan_suffixes([5, 9])
        with pytest.raises(BackendError):  # empty prefix
            pool.decode_step_shared_prefix(0, sp, None, None, q, _i32([]), _i32([0, 1, 2]), _i32([2, 3]))
        sp.close()
    for bad in (PoolDesc(1, 2, 14, 64, 8, "f32"), PoolDesc(1, 2, 8, 32, 8, "bf16")):
        with DeviceKvPool(bad) as pool:
            dt = torch.float32 if bad.dtype == "f32" else torch.bfloat16
            q = torch.zeros((2, bad.num_q_heads, bad.head_dim), dtype=dt, device="cuda")
            sp = pool.plan_suffixes([5, 9])
            with pytest.raises(BackendError):  # f32 pools / head_dim 32 have no MFMA tiles
                pool.decode_step_shared_prefix(0, sp, None, None, q, _i32([0]), _i32([0, 1, 2]), _i32([2, 3]))
            sp.close()


def test_shared_prefix_beside_and_in_order_agree():
    """A suffix plan built with pieces = 0 runs the prefix tiles beside the
    suffixes on the pool's second stream where the geometry allows it (one
    piece per CU); an explicit piece count runs the three launches in
    order. Back-to-back steps with different queries on one stream, no
    synchronisation between them, both forms against the oracle."""
    import torch

    L, Hq, Hkv, D = SHAPES["qwen7b"]
    seqs, prefix = 96, 4100
    batch = wl.shared_prefix_batch(seqs, prefix, 64, 700, wl.SplitMix64(127))
    full = prefix // 16
    sptr, sids, slen = _split_tables(batch, full)
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, "bf16")
    host = normal(128, desc.shape, "bf16")
    qs = [normal(129 + i, (seqs, Hq, D), "bf16") for i in range(3)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    got = {}
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        pre, sp_, si_ = _i32(batch.meta["shared_blocks"]), _i32(sptr), _i32(sids)
        for name, pieces in (("beside", 0), ("in_order", 2 * cus)):
            plan = pool.plan_suffixes(slen, pieces=pieces)
            if pieces == 0:
                assert plan.info()["pieces"] <= cus
            outs = [pool.decode_step_shared_prefix(L - 1, plan, None, None, to_device(q), pre, sp_, si_) for q in qs]
            pool.check()
            got[name] = [to_host(o) for o in outs]
            plan.close()
    for i, q in enumerate(qs):
        ref = orc.decode_attention(odesc(desc), host, L - 1, widen(q), batch.block_indptr, batch.block_ids,
                                   batch.ctx_lens)
        assert_attention_close(got["beside"][i], ref, "bf16")
        assert_attention_close(got["in_order"][i], ref, "bf16")
