"""Pins of the oracle's KV block wire format (payload layout and sum64
checksum, include/mitten_kv.h) and CPU tests of the header and message
framing (mitten_amd.wire; pure host code, no device).

The format has no reference implementation (the reference hands pages over
by index, design/phase2b-deliverable.md:272-289, and sketches per-layer SSD
KV files, design/phase1-deliverable.md:253-339), so it is pinned by what
its definition fixes:
* the checksum against a pure-Python big-integer restatement and the
  generator's published first output;
* the layout against numpy transposition of the pool;
* round trips between pools;
* the detection properties the checksum promises (every single-bit change,
  word swaps, block-local word index);
* mistakes planted in copies of the restatements, which all fail.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def _mix(z):
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _py_sum64(block: bytes, *, first_index=1, combine="add", word_offset=0):
    """Pure-Python restatement; keyword arguments plant mistakes."""
    acc = 0
    for j in range(len(block) // 8):
        w = int.from_bytes(block[8 * j:8 * j + 8], "little")
        m = _mix(w + (j + word_offset + first_index) * GOLDEN)
        acc = (acc + m) & M64 if combine == "add" else acc ^ m
    return acc


def _u(x):  # int64 bit pattern -> unsigned
    return int(np.int64(x)) & M64


def _pool(L, H, D, nb, es, seed):
    d = orc.desc(L, H, D, nb, es)
    raw = np.random.default_rng(seed).integers(0, 256, orc.pool_bytes(d), dtype=np.uint8)
    return d, raw.view(np.float32 if es == 4 else np.uint16).reshape(orc.pool_shape(d))


def test_sum64_known_answers():
    # one zero word: mix(golden), the first splitmix64 output of seed 0
    assert _u(orc.wire_checksums(np.zeros(8, np.uint8), 1, 8)[0]) == 0xE220A8397B1DCDAF
    # k zero words: the first k outputs of splitmix64 from seed 0, summed
    r = orc.SplitMix64(0)
    expect = 0
    for _ in range(64):
        expect = (expect + r.next()) & M64
    assert _u(orc.wire_checksums(np.zeros(512, np.uint8), 1, 512)[0]) == expect


def test_sum64_against_python_restatement():
    rng = np.random.default_rng(1)
    for nbytes in (8, 64, 1024, 4096):
        buf = rng.integers(0, 256, 3 * nbytes, dtype=np.uint8)
        got = orc.wire_checksums(buf, 3, nbytes)
        for i in range(3):
            assert _u(got[i]) == _py_sum64(buf[i * nbytes:(i + 1) * nbytes].tobytes())


def test_sum64_detects_changes():
    rng = np.random.default_rng(2)
    buf = rng.integers(0, 256, 2048, dtype=np.uint8)
    base = _u(orc.wire_checksums(buf, 1, 2048)[0])
    for bit in rng.choice(2048 * 8, 200, replace=False):  # every single-bit flip
        b = buf.copy()
        b[bit // 8] ^= np.uint8(1 << (bit % 8))
        assert _u(orc.wire_checksums(b, 1, 2048)[0]) != base
    words = buf.view(np.uint64).copy()
    for i, j in rng.integers(0, words.size, (50, 2)):  # word swaps
        if words[i] == words[j]:
            continue
        w = words.copy()
        w[i], w[j] = w[j], w[i]
        assert _u(orc.wire_checksums(w.view(np.uint8), 1, 2048)[0]) != base
    # the word index is block-local: the same block gives the same sum anywhere in a message
    two = np.concatenate([rng.integers(0, 256, 2048, dtype=np.uint8), buf])
    assert _u(orc.wire_checksums(two, 2, 2048)[1]) == base


@pytest.mark.parametrize("es", [4, 2])
def test_export_layout_is_the_block_major_transpose(es):
    L, H, D, nb = 4, 2, 32, 9
    d, pool = _pool(L, H, D, nb, es, 3)
    ids = np.array([7, 0, 3, 3, 8], np.int32)
    for lb, nl in ((0, 4), (1, 2), (3, 1)):
        payload, sums = orc.wire_export(d, pool, ids, lb, nl)
        expect = np.ascontiguousarray(pool[lb:lb + nl][:, :, ids].transpose(2, 0, 1, 3, 4, 5))
        assert np.array_equal(payload, expect.reshape(-1).view(np.uint8))
        per = nl * 2 * 16 * H * D * es
        for i in range(ids.size):
            assert _u(sums[i]) == _py_sum64(payload[i * per:(i + 1) * per].tobytes())
    with pytest.raises(ValueError):
        orc.wire_export(d, pool, np.array([1, nb], np.int32), 0, 1)


def test_round_trip_between_pools():
    L, H, D, nb = 3, 2, 64, 12
    d, a = _pool(L, H, D, nb, 2, 4)
    _, b = _pool(L, H, D, nb, 2, 5)
    src, dst = np.array([2, 9, 4], np.int32), np.array([11, 0, 5], np.int32)
    b0 = b.copy()
    payload, sums = orc.wire_export(d, a, src, 1, 2)
    got = orc.wire_import(d, b, dst, 1, 2, payload)
    assert np.array_equal(got, sums)
    assert np.array_equal(b[1:3][:, :, dst], a[1:3][:, :, src])
    keep = np.ones(b.shape[:3], bool)
    keep[1:3, :, dst] = False
    assert np.array_equal(b[keep], b0[keep])  # layer 0 and the other blocks untouched


def test_checks_detect_planted_mistakes():
    L, H, D, nb = 2, 2, 32, 6
    d, pool = _pool(L, H, D, nb, 2, 6)
    ids = np.array([5, 1, 2], np.int32)
    payload, sums = orc.wire_export(d, pool, ids, 0, 2)
    per = 2 * 2 * 16 * H * D * 2
    blk1 = payload[per:2 * per].tobytes()
    assert _u(sums[1]) == _py_sum64(blk1)
    wrong_sums = {
        "index from 0": _py_sum64(blk1, first_index=0),
        "xor instead of add": _py_sum64(blk1, combine="xor"),
        "message-global word index": _py_sum64(blk1, word_offset=per // 8),
    }
    for name, w in wrong_sums.items():
        assert w != _u(sums[1]), name
    layer_major = np.ascontiguousarray(pool[:, :, ids].transpose(0, 1, 2, 3, 4, 5)).reshape(-1).view(np.uint8)
    kv_inner = np.ascontiguousarray(pool[:, :, ids].transpose(2, 1, 0, 3, 4, 5)).reshape(-1).view(np.uint8)
    for name, w in {"layer-major": layer_major, "K/V outside layers": kv_inner}.items():
        assert not np.array_equal(w, payload), name


# ---- header and framing (host code in the device library; no device) ---------------------

def test_header_init_and_check():
    from mitten_amd import PoolDesc, _lib
    from mitten_amd import wire

    lib = _lib.device_lib()
    desc = PoolDesc(28, 4, 28, 128, 1000, "bf16")
    h = _lib.WireHeaderC()
    assert lib.mkv_wire_header_init(ctypes.byref(desc.c()), 0, 28, 300, 4700, ctypes.byref(h)) == 0
    assert ctypes.sizeof(h) == wire.HEADER_BYTES == 64
    raw = bytes(h)
    assert raw[:4] == b"MKVW" and h.version == 1 and h.dtype == 1
    assert h.block_bytes == 28 * 2 * 16 * 4 * 128 * 2
    assert h.payload_offset % 4096 == 0 and h.payload_offset >= 64 + 8 * 300
    assert lib.mkv_wire_header_check(ctypes.byref(desc.c()), ctypes.byref(h)) == 0
    # another geometry, a newer version, a foreign magic, a layer range past the pool
    for field, value in (("head_dim", 64), ("version", 2), ("magic", 0), ("num_layers", 29)):
        bad = _lib.WireHeaderC.from_buffer_copy(raw)
        setattr(bad, field, value)
        assert lib.mkv_wire_header_check(ctypes.byref(desc.c()), ctypes.byref(bad)) != 0, field
    assert lib.mkv_wire_header_init(ctypes.byref(desc.c()), 0, 1, 2, 33, ctypes.byref(h)) != 0  # 33 > 2 * 16


def test_message_encode_decode():
    from mitten_amd import PoolDesc, _lib
    from mitten_amd import wire

    desc = PoolDesc(2, 1, 8, 32, 10, "f32")
    h = _lib.WireHeaderC()
    assert _lib.device_lib().mkv_wire_header_init(ctypes.byref(desc.c()), 1, 1, 3, 40, ctypes.byref(h)) == 0
    payload = np.random.default_rng(7).integers(0, 256, 3 * h.block_bytes, dtype=np.uint8)
    sums = orc.wire_checksums(payload, 3, h.block_bytes)
    msg = wire.encode(h, sums, payload.tobytes())
    assert len(msg) == h.payload_offset + payload.size
    h2, s2, p2 = wire.decode(msg)
    assert bytes(h2) == bytes(h) and np.array_equal(s2, sums) and bytes(p2) == payload.tobytes()
    with pytest.raises(Exception):
        wire.decode(msg[:-1])
