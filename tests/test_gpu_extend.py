"""GPU parity of extend (chunked prefill) attention through the C ABI:
each sequence's newest tokens attend causally over the whole cache,
against the oracle (bf16 row-relative 2e-2, f32 max-abs 1e-5), plus the
identities the oracle tests pin (the chunk's last query equals decode
attention) and the error paths. Both paths: MFMA query tiles (bf16,
head_dim 64/128/256, up to 16 query heads per KV head) and per-token
decode segments (everything else)."""
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
    # name: (Hq, Hkv, D): query heads per KV head G = 7, 8, 7, 4, 16, 1, 4, 16
    "qwen7b": (28, 4, 128),
    "gemma2b": (8, 1, 256),
    "qwen0.5b": (14, 2, 64),
    "llama8b": (32, 8, 128),
    "g16": (64, 4, 128),
    "mha": (4, 4, 64),
    "d256-g4": (16, 4, 256),   # head_dim 256 with 4 waves per workgroup
    "d256-g16": (16, 1, 256),  # head_dim 256 with 16 waves per workgroup
}
# Shapes the MFMA tile kernel does not take (per-token segments instead).
SEGMENT_SHAPES = {
    # name: (Hq, Hkv, D, dtype)
    "qwen0.5b-f32": (14, 2, 64, "f32"),   # the reference's CPU-runnable configuration
    "d32-f32": (8, 4, 32, "f32"),
    "d128-f32": (28, 4, 128, "f32"),
    "g32-bf16": (64, 2, 128, "bf16"),     # 32 query heads per KV head
    "d32-bf16": (8, 2, 32, "bf16"),
}


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _case(shape, ctx, nq, seed, zero_sink=False, layer=1, dtype="bf16"):
    """shape: a SHAPES name or an (Hq, Hkv, D) tuple."""
    Hq, Hkv, D = SHAPES[shape] if isinstance(shape, str) else shape
    rng = wl.SplitMix64(seed)
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng, extra_blocks=2)
    desc = PoolDesc(2, Hkv, Hq, D, batch.num_blocks, dtype)
    host = normal(seed + 1, desc.shape, dtype)
    q_indptr = np.concatenate([[0], np.cumsum(nq)]).astype(np.int32)
    q = normal(seed + 2, (int(q_indptr[-1]), Hq, D), dtype)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        o = pool.extend_attention(layer, to_device(q), _i32(q_indptr), _i32(batch.block_indptr),
                                  _i32(batch.block_ids), _i32(batch.ctx_lens), max(nq), max(ctx),
                                  zero_sink=zero_sink)
        pool.check()
        got = to_host(o)
        dec = None
        if not zero_sink:  # the last query of each chunk is a decode query over the whole context
            last = q_indptr[1:] - 1
            dec = to_host(pool.decode_attention(layer, to_device(q[last]), _i32(batch.block_indptr),
                                                _i32(batch.block_ids), _i32(batch.ctx_lens), max(ctx)))
    ref = orc.extend_attention(odesc(desc), host, layer, widen(q), q_indptr, batch.block_indptr,
                               batch.block_ids, batch.ctx_lens, zero_sink=zero_sink)
    return got, ref, dec, q_indptr


CTX = [1, 16, 17, 40, 200, 530, 97]
NQ = [1, 16, 5, 40, 33, 512, 1]  # whole prompts, chunks after a prefix, a single token


@pytest.mark.parametrize("shape", list(SHAPES))
def test_extend_attention_matches_oracle(shape):
    got, ref, dec, q_indptr = _case(shape, CTX, NQ, 90)
    assert_attention_close(got, ref, "bf16")
    last = q_indptr[1:] - 1
    assert_attention_close(dec, ref[last], "bf16")


def test_extend_attention_zero_sink():
    got, ref, _, _ = _case("qwen7b", [1, 20, 300], [1, 20, 64], 91, zero_sink=True)
    assert_attention_close(got, ref, "bf16")


@pytest.mark.parametrize("shape", ["qwen7b", "qwen0.5b", "mha"])
def test_extend_short_chunks(shape):
    """Chunks of at most 16 tokens (one query sub-tile per workgroup) after
    prefixes of assorted lengths."""
    got, ref, dec, q_indptr = _case(shape, [16, 300, 1000, 47, 8], [16, 1, 9, 16, 3], 97)
    assert_attention_close(got, ref, "bf16")
    assert_attention_close(dec, ref[q_indptr[1:] - 1], "bf16")


def test_extend_long_context_chunk():
    """A 512-token chunk at the end of an 8k context (the pool-pressure
    configuration's chunked prefill)."""
    got, ref, _, _ = _case("qwen7b", [8192, 700], [512, 64], 92)
    assert_attention_close(got, ref, "bf16")


def test_extend_key_range_past_the_staged_ids():
    """A workgroup whose key range holds more blocks than the kernel stages
    in LDS for its unmasked steps (1,024 ids) takes the generic step
    throughout: one 16-token chunk at the end of a 16,900-token context
    (1,057 blocks), beside 255 short prompts so that the launch fills the
    device and the long range is not split."""
    ctx = [16900] + [16] * 255
    nq = [16] * 256
    got, ref, dec, q_indptr = _case("qwen7b", ctx, nq, 98)
    assert_attention_close(got, ref, "bf16")
    assert_attention_close(dec, ref[q_indptr[1:] - 1], "bf16")


def test_extend_errors_are_reported():
    Hq, Hkv, D = SHAPES["qwen7b"]
    desc = PoolDesc(1, Hkv, Hq, D, 10, "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(normal(93, desc.shape, "bf16"))
        q = to_device(normal(94, (4, Hq, D), "bf16"))
        qi = _i32([0, 2, 4])
        # block id outside the pool
        pool.extend_attention(0, q, qi, _i32([0, 2, 4]), _i32([1, 2, 3, 10]), _i32([20, 30]), 2, 30)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_BLOCK
        # table too short for the context
        pool.extend_attention(0, q, qi, _i32([0, 1, 3]), _i32([1, 2, 3]), _i32([20, 30]), 2, 30)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_TABLE
        # context beyond max_ctx_len
        pool.extend_attention(0, q, qi, _i32([0, 2, 4]), _i32([1, 2, 3, 4]), _i32([20, 30]), 2, 25)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_CTX
        with pytest.raises(BackendError):  # max_q_len > max_ctx_len
            pool.extend_attention(0, q, qi, _i32([0, 2, 4]), _i32([1, 2, 3, 4]), _i32([20, 30]), 40, 30)
    f32 = PoolDesc(1, 2, 14, 64, 4, "f32")
    with DeviceKvPool(f32) as pool:
        import torch

        q = torch.zeros((2, 14, 64), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(BackendError):  # q must be in the pool dtype
            pool.extend_attention(0, q, _i32([0, 2]), _i32([0, 1]), _i32([0]), _i32([2]), 2, 2)


def test_extend_split_key_ranges_with_empty_splits():
    """Few sequences over long contexts split each key range (f32 partials,
    then a merge); short contexts in the same launch leave some splits with
    no blocks, which must merge as empty partials."""
    got, ref, dec, q_indptr = _case("qwen7b", [3000, 1, 17, 6000, 40], [16, 1, 3, 12, 40], 98)
    assert_attention_close(got, ref, "bf16")
    assert_attention_close(dec, ref[q_indptr[1:] - 1], "bf16")


def test_extend_split_rejects_chunk_past_max_q_len():
    """With split key ranges a chunk longer than max_q_len is reported
    (its partial rows would lie past the workspace), not written."""
    Hq, Hkv, D = SHAPES["qwen7b"]
    rng = wl.SplitMix64(99)
    batch = wl.decode_batch_from_contexts([2000 - 1], rng, extra_blocks=2)
    desc = PoolDesc(1, Hkv, Hq, D, batch.num_blocks, "bf16")
    with DeviceKvPool(desc) as pool:
        pool.write(normal(99, desc.shape, "bf16"))
        q = to_device(normal(100, (20, Hq, D), "bf16"))
        pool.extend_attention(0, q, _i32([0, 20]), _i32(batch.block_indptr), _i32(batch.block_ids),
                              _i32(batch.ctx_lens), 16, 2000)
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_CTX


@pytest.mark.parametrize("name", list(SEGMENT_SHAPES))
def test_extend_segment_path_matches_oracle(name):
    """f32 pools, head_dim 32 and groups above 16 run one decode segment per
    query token: f32 within max-abs 1e-5, bf16 within row-relative 2e-2."""
    Hq, Hkv, D, dt = SEGMENT_SHAPES[name]
    ctx, nq = [1, 17, 40, 300, 97], [1, 17, 25, 64, 1]
    got, ref, dec, q_indptr = _case((Hq, Hkv, D), ctx, nq, 95, dtype=dt)
    assert_attention_close(got, ref, dt)
    assert_attention_close(dec, ref[q_indptr[1:] - 1], dt)
    got, ref, _, _ = _case((Hq, Hkv, D), [50, 33], [20, 33], 96, zero_sink=True, dtype=dt)
    assert_attention_close(got, ref, dt)
