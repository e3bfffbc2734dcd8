"""The C ABI libraries load without a GPU and export every function that
include/*.h declares; host-side validation works with no device access."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from mitten_amd import BackendError, PoolDesc, _build, required_bytes, validate_block_tables
from mitten_amd import validate_copy_pairs, validate_slots

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str, prefix: str):
    text = open(os.path.join(ROOT, "include", header)).read()
    api = prefix.upper() + "_API"
    return sorted(set(re.findall(rf"{api}[^;(]*?\b({prefix}_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib,prefix", [
    ("mitten_kv.h", _build.DEVICE_LIB, "mkv"),
    ("mitten_kv_host.h", _build.HOST_LIB, "mkvh"),
])
def test_library_exports_every_declared_symbol(header, lib, prefix):
    names = _declared(header, prefix)
    assert len(names) > 10
    so = ctypes.CDLL(lib)
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, f"{os.path.basename(lib)} lacks {missing}"


def test_python_bindings_cover_the_header():
    from mitten_amd import _host_sigs, _lib

    assert set(_declared("mitten_kv.h", "mkv")) == set(_lib.DEVICE_SIGNATURES)
    assert set(_declared("mitten_kv_host.h", "mkvh")) == set(_host_sigs.HOST_SIGNATURES)


def test_version_through_the_abi():
    from mitten_amd import _lib

    assert _lib.device_lib().mkv_version() == 100  # 0.1.0 as MAJOR*10000 + MINOR*100 + PATCH


def test_required_bytes_reference_kat_through_the_abi():
    # kv_pool.rs:130-136
    assert required_bytes(PoolDesc(28, 4, 28, 128, 512, "bf16")) == 469_762_048


@pytest.mark.parametrize("bad", [
    dict(num_layers=0), dict(num_kv_heads=3, num_q_heads=28), dict(head_dim=12), dict(head_dim=1024),
    dict(page_size=8), dict(dtype="fp8"), dict(num_blocks=0),
])
def test_descriptor_validation(bad):
    kw = dict(num_layers=2, num_kv_heads=4, num_q_heads=28, head_dim=128, num_blocks=10, dtype="bf16")
    kw.update(bad)
    with pytest.raises((BackendError, KeyError)):
        required_bytes(PoolDesc(**kw))


def test_host_validators():
    d = PoolDesc(2, 4, 28, 128, 10, "bf16")
    validate_slots(d, [0, 159])
    for bad in ([160], [-1]):
        with pytest.raises(BackendError):
            validate_slots(d, bad)
    validate_block_tables(d, [0, 2, 3], [1, 2, 9], [17, 16], 17)
    with pytest.raises(BackendError):  # table of sequence 0 too short for 33 tokens
        validate_block_tables(d, [0, 2, 3], [1, 2, 9], [33, 16], 33)
    with pytest.raises(BackendError):  # block id out of range
        validate_block_tables(d, [0, 1], [10], [5], 5)
    with pytest.raises(BackendError):  # context longer than max_ctx_len
        validate_block_tables(d, [0, 2], [1, 2], [20], 16)
    with pytest.raises(BackendError) as ei:  # indptr falls back: refused before ids past the end are read
        validate_block_tables(d, [0, 40, 2], [1, 2], [600, 20], 600)
    assert "not monotone at 1" in str(ei.value)
    validate_copy_pairs(d, [1, 2], [3, 4])
    for src, dst in (([1, 2], [2, 3]), ([1, 2], [3, 3]), ([1], [10])):
        with pytest.raises(BackendError):
            validate_copy_pairs(d, src, dst)


def test_pool_create_without_device_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    from mitten_amd import DeviceKvPool

    with pytest.raises(BackendError) as ei:
        DeviceKvPool(PoolDesc(1, 1, 1, 64, 4, "f32"))
    assert ei.value.status == 5  # MKV_ERR_NO_DEVICE


def test_last_error_is_thread_local_and_descriptive():
    from mitten_amd import _lib

    lib = _lib.device_lib()
    d = PoolDesc(2, 4, 28, 128, 10, "bf16").c()
    s = np.array([999], np.int32)
    assert lib.mkv_validate_slots(ctypes.byref(d), s.ctypes.data_as(_lib.I32P), 1) == 1
    assert b"slot[0] = 999" in lib.mkv_last_error()


@pytest.mark.parametrize("bad,msg", [(np.array([3, 2**32 + 5], np.int64), "2^32"),
                                     (np.array([2**32], np.uint64), "2^32"),
                                     (np.array([4, -1], np.int32), "negative"),
                                     (np.array([1.5]), "integers")])
def test_host_u32_metadata_refuses_values_outside_u32(bad, msg):
    """Engine ids and slots are u32: 2^32 + 5 must not wrap to slot 5 (a
    valid slot of another sequence), and negative or fractional values are
    not ids."""
    from mitten_amd import device_pool as dp

    for name in ("slot_mapping", "block_ids"):
        with pytest.raises(BackendError) as ei:
            dp._host_u32(bad, name)
        assert ei.value.status == dp.MKV_ERR_INVALID_ARGUMENT
        assert name in str(ei.value) and msg in str(ei.value)
    assert dp._host_u32(np.array([0, 2**32 - 1], np.int64), "ids").tolist() == [0, 2**32 - 1]
    assert dp._host_u32([], "ids").size == 0


@pytest.mark.parametrize("bad,msg", [(np.array([7, 2**32 + 5], np.int64), "outside int32"),
                                     (np.array([2**31], np.int64), "outside int32"),
                                     (np.array([-2**31 - 1], np.int64), "outside int32"),
                                     (np.array([2.0]), "integers")])
def test_host_i32_metadata_refuses_values_outside_i32(bad, msg):
    """Context lengths, positions and the validators' ids are i32: 2^32 + 5
    must not wrap to 5, which would pass every later check."""
    from mitten_amd import device_pool as dp

    with pytest.raises(BackendError) as ei:
        dp._host_i32(bad, "ctx_lens")
    assert ei.value.status == dp.MKV_ERR_INVALID_ARGUMENT
    assert "ctx_lens" in str(ei.value) and msg in str(ei.value)
    desc = PoolDesc(2, 4, 28, 128, 10, "bf16")
    with pytest.raises(BackendError):
        dp.validate_slots(desc, bad)
    with pytest.raises(BackendError):
        dp.validate_copy_pairs(desc, bad, bad)
    assert dp._host_i32(np.array([-2**31, 2**31 - 1], np.int64), "x").tolist() == [-2**31, 2**31 - 1]
    assert dp._host_i32([], "x").size == 0


@pytest.mark.parametrize("bad", [np.array([5, 2**32 + 1], np.int64), np.array([-1], np.int64), np.array([0.5])])
def test_host_library_refuses_token_and_page_ids_outside_u32(bad):
    """The radix tree's token ids and page ids are u32 (radix_cache.rs:37-62):
    a value outside u32 is refused, not wrapped into another token or page."""
    from mitten_amd.host import INVALID_ARGUMENT, HostError, RadixCache

    rc = RadixCache(16, 8)
    with pytest.raises(HostError) as ei:
        rc.insert_prefix(bad, np.arange(1))
    assert ei.value.status == INVALID_ARGUMENT and "tokens" in str(ei.value)
    with pytest.raises(HostError) as ei:
        rc.insert_prefix(np.arange(16 * bad.size), bad)
    assert ei.value.status == INVALID_ARGUMENT and "pages" in str(ei.value)
    with pytest.raises(HostError):
        rc.match_prefix(bad)
