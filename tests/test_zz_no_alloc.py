"""The no-allocation decode entry point (mkv_decode_attention_static): split-K
partials in the library's static device scratch instead of a workspace.

Through the C ABI it must give the same bits as mkv_decode_attention with a
caller workspace and the same split, on two calls in a row (the second with a
smaller batch, over the scratch the first one left behind), allocate no
device memory, and refuse an explicit split whose partials exceed the
scratch (before anything is launched)."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import BackendError, DeviceKvPool, PoolDesc
from mitten_amd import device_pool as dp
from mitten_amd import workloads as wl
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _both(pool, desc, batch, q, split_tokens, kernel=None):
    """(static output, workspace output) of one layer-0 decode."""
    import torch

    ip, ix, cl = _i32(batch.block_indptr), _i32(batch.block_ids), _i32(batch.ctx_lens)
    ws = torch.empty(max(1, pool.workspace_size(batch.num_seqs, batch.max_ctx, split_tokens)), dtype=torch.uint8,
                     device="cuda")
    o_ws = pool.decode_attention(0, to_device(q), ip, ix, cl, batch.max_ctx, split_tokens=split_tokens, workspace=ws,
                                 kernel=kernel)
    o_st = pool.decode_attention_static(0, to_device(q), ip, ix, cl, batch.max_ctx, split_tokens=split_tokens,
                                       kernel=kernel)
    pool.check()
    return to_host(o_st), to_host(o_ws)


@pytest.mark.parametrize("shape,kernel", [((28, 4, 128, "bf16"), None), ((28, 4, 128, "bf16"), "valu"),
                                          ((8, 1, 256, "bf16"), None), ((14, 2, 64, "f32"), None)])
def test_static_scratch_matches_workspace_entry_on_two_calls(shape, kernel):
    import torch

    Hq, Hkv, D, dt = shape
    rng = wl.SplitMix64(300)
    big = wl.decode_batch_from_contexts(wl.uniform_contexts(64, 1000, 4095, rng), rng, extra_blocks=8)
    small = wl.decode_batch_from_contexts([5, 300, 17, 900, 64], wl.SplitMix64(301), extra_blocks=2)
    n = max(big.num_blocks, small.num_blocks)
    desc = PoolDesc(1, Hkv, Hq, D, n, dt)
    host = normal(302, desc.shape, dt)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        torch.cuda.synchronize()
        for batch, seed, st in ((big, 303, 0), (small, 304, 0), (big, 305, 128), (small, 306, 32)):
            q = normal(seed, (batch.num_seqs, Hq, D), dt)
            got, want = _both(pool, desc, batch, q, st, kernel)
            assert np.array_equal(bits(got), bits(want)), f"static differs from workspace (B={batch.num_seqs})"
            ref = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids,
                                       batch.ctx_lens)
            assert_attention_close(got, ref, dt)


def test_static_scratch_allocates_no_device_memory():
    """Partials of ~15 MB per call: an allocation of them would show in the
    device's free memory; the free memory does not move."""
    import torch

    Hq, Hkv, D = 28, 4, 128
    rng = wl.SplitMix64(310)
    batch = wl.decode_batch_from_contexts(wl.uniform_contexts(64, 3000, 8191, rng), rng)
    desc = PoolDesc(1, Hkv, Hq, D, batch.num_blocks, "bf16")
    q = to_device(normal(311, (batch.num_seqs, Hq, D), "bf16"))
    ip, ix, cl = _i32(batch.block_indptr), _i32(batch.block_ids), _i32(batch.ctx_lens)
    assert pool_partials_bytes(desc, batch) > 8 << 20
    with DeviceKvPool(desc) as pool:
        out = torch.empty_like(q)
        out.zero_()  # the stream's first kernel launch is torch's, not the entry point's
        # The pool's creation already loaded the code objects (it looks up the
        # scratch's address), so the baseline is taken before the first call:
        # an allocation on the first call, or growth across calls, both show.
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        for _ in range(4):
            pool.decode_attention_static(0, q, ip, ix, cl, batch.max_ctx, out=out)
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        pool.check()
    assert free0 - free1 < 4 << 20, f"device free memory fell by {free0 - free1} bytes"


def pool_partials_bytes(desc, batch):
    """Bytes of the split-K partials the library's automatic split gives
    (the workspace size query of the workspace entry point)."""
    import torch  # noqa: F401

    with DeviceKvPool(PoolDesc(1, desc.num_kv_heads, desc.num_q_heads, desc.head_dim, 1, desc.dtype)) as p:
        return p.workspace_size(batch.num_seqs, batch.max_ctx, 0)


def test_static_scratch_refuses_an_explicit_split_beyond_it():
    """split_tokens = 16 over 4k contexts: 64 x 28 x 256 partial rows (238 MB)
    exceed the 64 MiB scratch; refused on the host, the output untouched. The
    library's own split at the same size fits and is computed."""
    import torch

    Hq, Hkv, D = 28, 4, 128
    rng = wl.SplitMix64(320)
    batch = wl.decode_batch_from_contexts([4095] * 64, rng)
    desc = PoolDesc(1, Hkv, Hq, D, batch.num_blocks, "bf16")
    host = normal(321, desc.shape, "bf16")
    q = normal(322, (batch.num_seqs, Hq, D), "bf16")
    ip, ix, cl = _i32(batch.block_indptr), _i32(batch.block_ids), _i32(batch.ctx_lens)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        out = torch.full((batch.num_seqs, Hq, D), 7.0, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(BackendError) as ei:
            pool.decode_attention_static(0, to_device(q), ip, ix, cl, batch.max_ctx, split_tokens=16, out=out)
        assert ei.value.status == dp.MKV_ERR_INVALID_ARGUMENT and "scratch" in str(ei.value)
        torch.cuda.synchronize()
        assert bool((out == 7.0).all())
        got = to_host(pool.decode_attention_static(0, to_device(q), ip, ix, cl, batch.max_ctx))
        pool.check()
    ref = orc.decode_attention(odesc(desc), host, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens)
    assert_attention_close(got, ref, "bf16")
