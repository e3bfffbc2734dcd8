"""GPU parity of the KV block wire format (mkv_wire_export / mkv_wire_import)
against the oracle, bit-exact: payload bytes, per-block checksums, and the
pool after an import; message round trips between pools through host bytes;
corruption, bad ids and foreign headers reported."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import BackendError, DeviceIndexError, DeviceKvPool, PoolDesc
from mitten_amd import device_pool as dp
from mitten_amd import wire
from oracle import oracle as orc
from tests.helpers import odesc, to_host

pytestmark = pytest.mark.gpu

SHAPES = {
    # name: (layers, Hkv, Hq, D, dtype)
    "qwen7b": (28, 4, 28, 128, "bf16"),
    "qwen0.5b-f32": (24, 2, 14, 64, "f32"),
    "gemma2b": (18, 1, 8, 256, "bf16"),
}


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _random_pool(desc, seed):
    raw = np.random.default_rng(seed).integers(0, 256, int(np.prod(desc.shape)) * desc.elem_bytes,
                                               dtype=np.uint8)
    return raw.view(np.uint32 if desc.dtype == "f32" else np.uint16).reshape(desc.shape)


def _read(pool):
    """The pool as bit patterns (random f32 bytes include NaNs)."""
    a = pool.read()
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("shape", list(SHAPES))
def test_export_matches_oracle(shape):
    L, Hkv, Hq, D, dt = SHAPES[shape]
    desc = PoolDesc(L, Hkv, Hq, D, 40, dt)
    host = _random_pool(desc, 1)
    ids = np.array([39, 0, 17, 17, 5, 22, 1], np.int32)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        for lb, nl in ((0, L), (L - 1, 1), (3, 5)):
            payload, sums = pool.wire_export(_i32(ids), lb, nl)
            pool.check()
            ref_p, ref_s = orc.wire_export(odesc(desc), host, ids, lb, nl)
            assert np.array_equal(to_host(payload), ref_p), (lb, nl)
            assert np.array_equal(to_host(sums), ref_s), (lb, nl)


@pytest.mark.parametrize("shape", ["qwen7b", "qwen0.5b-f32"])
def test_import_matches_oracle(shape):
    L, Hkv, Hq, D, dt = SHAPES[shape]
    desc = PoolDesc(L, Hkv, Hq, D, 30, dt)
    src_host, dst_host = _random_pool(desc, 2), _random_pool(desc, 3)
    src, dst = np.array([4, 9, 28, 0], np.int32), np.array([29, 3, 11, 12], np.int32)
    payload, sums = orc.wire_export(odesc(desc), src_host, src, 2, L - 2)
    import torch

    with DeviceKvPool(desc) as pool:
        pool.write(dst_host)
        got = pool.wire_import(_i32(dst), torch.from_numpy(payload).cuda(), 2, L - 2,
                               expected=torch.from_numpy(sums.copy()).cuda())
        pool.check()
        after = _read(pool)
    ref = dst_host.copy()
    ref_s = orc.wire_import(odesc(desc), ref, dst, 2, L - 2, payload)
    assert np.array_equal(after, ref)
    assert np.array_equal(to_host(got), ref_s)


def test_message_round_trip_between_pools():
    """A request's pages leave one pool as bytes and enter another at other
    block ids: every carried plane bit-identical, the rest untouched."""
    L, Hkv, Hq, D, dt = SHAPES["qwen7b"]
    desc_a = PoolDesc(L, Hkv, Hq, D, 64, dt)
    desc_b = PoolDesc(L, Hkv, Hq, D, 80, dt)
    a_host, b_host = _random_pool(desc_a, 4), _random_pool(desc_b, 5)
    pages = np.array([63, 2, 40, 7, 8], np.int32)  # 5 pages, 70 tokens
    dest = np.array([0, 79, 41, 3, 50], np.int32)
    with DeviceKvPool(desc_a) as pa, DeviceKvPool(desc_b) as pb:
        pa.write(a_host)
        pb.write(b_host)
        msg = wire.export_blocks(pa, pages, cached_len=70)
        h = wire.import_blocks(pb, msg, dest)
        b_after = pb.read()
    assert h.cached_len == 70 and h.num_blocks == 5 and h.num_layers == L
    assert np.array_equal(b_after[:, :, dest], a_host[:, :, pages])
    keep = np.ones(b_after.shape[:3], bool)
    keep[:, :, dest] = False
    assert np.array_equal(b_after[keep], b_host[keep])


def test_one_layer_offload_chunk():
    """num_layers = 1: the per-layer offload chunk; writing it back restores
    the layer after it was overwritten."""
    L, Hkv, Hq, D, dt = SHAPES["gemma2b"]
    desc = PoolDesc(L, Hkv, Hq, D, 50, dt)
    host = _random_pool(desc, 6)
    ids = np.arange(50, dtype=np.int32)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        msg = wire.export_blocks(pool, ids, cached_len=800, layer_begin=6, num_layers=1)
        pool.write(np.zeros_like(host))
        wire.import_blocks(pool, msg, ids)
        after = pool.read()
    assert np.array_equal(after[6], host[6])
    assert not after[:6].any() and not after[7:].any()


def test_corruption_and_bad_ids_are_reported():
    import torch

    L, Hkv, Hq, D, dt = SHAPES["qwen0.5b-f32"]
    desc = PoolDesc(L, Hkv, Hq, D, 10, dt)
    host = _random_pool(desc, 7)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        msg = bytearray(wire.export_blocks(pool, [1, 2, 3], cached_len=40))
        h, _, _ = wire.decode(msg)
        msg[h.payload_offset + h.block_bytes + 12345] ^= 0x10  # one bit of block 1
        with pytest.raises(DeviceIndexError) as ei:
            wire.import_blocks(pool, bytes(msg), [4, 5, 6])
        assert ei.value.bits & dp.DEVERR_CHECKSUM
        # the checksums of the received bytes say which block differs
        payload, sums = pool.wire_export(_i32([1, 2, 3]))
        got = pool.wire_import(_i32([4, 5, 6]), torch.from_numpy(np.frombuffer(
            bytes(msg[h.payload_offset:]), np.uint8).copy()).cuda())
        pool.check()
        assert (to_host(got) != to_host(sums)).tolist() == [False, True, False]
        # a block id outside the pool
        pool.wire_export(_i32([1, 10]))
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_BLOCK
        # a message from a pool of another geometry
        other = PoolDesc(L, Hkv, Hq, 128, 10, dt)
        with DeviceKvPool(other) as po:
            with pytest.raises(BackendError):
                wire.import_blocks(po, bytes(msg), [4, 5, 6])
        with pytest.raises(BackendError):  # layer range past the pool
            pool.wire_export(_i32([1]), L - 1, 2)


def test_large_handoff_checksums():
    """300 Qwen-7B pages, all 28 layers (262 MB): the device checksums equal
    the oracle's checksums of the exported bytes, and 20 sampled blocks equal
    the pool."""
    L, Hkv, Hq, D, dt = SHAPES["qwen7b"]
    desc = PoolDesc(L, Hkv, Hq, D, 400, dt)
    rng = np.random.default_rng(8)
    ids = rng.permutation(400)[:300].astype(np.int32)
    with DeviceKvPool(desc) as pool:
        view = pool.tensor()
        import torch

        gen = torch.Generator(device="cuda")
        gen.manual_seed(8)
        for layer in range(L):
            view[layer].normal_(generator=gen)
        del view
        payload, sums = pool.wire_export(_i32(ids))
        pool.check()
        p_host, s_host = to_host(payload), to_host(sums)
        bb = pool.wire_block_bytes()
        sample = rng.choice(300, 20, replace=False)
        pool_host = pool.read()
    assert np.array_equal(orc.wire_checksums(p_host, 300, bb), s_host)
    for i in sample:
        blk = pool_host[:, :, ids[i]]
        assert np.array_equal(p_host[i * bb:(i + 1) * bb], np.ascontiguousarray(blk).reshape(-1).view(np.uint8))
