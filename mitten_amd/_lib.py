"""ctypes loading of libmitten_kv.so / libmitten_kvhost.so with full signatures.

No fallback: if a library is missing, loading raises MkvLibraryMissing, so a
caller can never silently run anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os

from . import _build

P = ctypes.c_void_p
i32, i64, u32, u64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
c_int = ctypes.c_int


class MkvLibraryMissing(RuntimeError):
    pass


class PoolDescC(ctypes.Structure):
    _fields_ = [
        ("num_layers", i32),
        ("num_kv_heads", i32),
        ("num_q_heads", i32),
        ("head_dim", i32),
        ("page_size", i32),
        ("dtype", i32),
        ("num_blocks", i64),
    ]


class WireHeaderC(ctypes.Structure):
    _fields_ = [
        ("magic", ctypes.c_uint32),
        ("version", ctypes.c_uint16),
        ("dtype", ctypes.c_uint16),
        ("page_size", i32),
        ("num_kv_heads", i32),
        ("head_dim", i32),
        ("layer_begin", i32),
        ("num_layers", i32),
        ("num_blocks", i32),
        ("cached_len", i64),
        ("block_bytes", u64),
        ("payload_offset", u64),
        ("reserved", u64),
    ]


DESC_P = ctypes.POINTER(PoolDescC)
WIRE_P = ctypes.POINTER(WireHeaderC)
I32P = ctypes.POINTER(i32)
U32P = ctypes.POINTER(u32)

DEVICE_SIGNATURES = {
    "mkv_pool_required_bytes": (c_int, [DESC_P, ctypes.POINTER(u64)]),
    "mkv_pool_create": (c_int, [DESC_P, c_int, ctypes.POINTER(P)]),
    "mkv_pool_destroy": (c_int, [P]),
    "mkv_pool_get_desc": (c_int, [P, DESC_P]),
    "mkv_pool_buffer": (c_int, [P, ctypes.POINTER(P), ctypes.POINTER(u64)]),
    "mkv_pool_check": (c_int, [P, P, ctypes.POINTER(u32)]),
    "mkv_pool_set_launch_events": (c_int, [P, P, P]),
    "mkv_append": (c_int, [P, i32, P, P, P, i32, P]),
    "mkv_append_all_layers": (c_int, [P, P, P, P, i32, P]),
    "mkv_gather": (c_int, [P, i32, P, P, P, i32, i32, P, P, i64, P]),
    "mkv_copy_blocks": (c_int, [P, P, P, i32, P]),
    "mkv_decode_attention": (c_int, [P, i32, P, P, P, P, P, i32, i32, f32, u32, i32, P, u64, P]),
    "mkv_decode_attention_workspace_size": (c_int, [P, i32, i32, i32, ctypes.POINTER(u64)]),
    "mkv_decode_attention_static": (c_int, [P, i32, P, P, P, P, P, i32, i32, f32, u32, i32, P]),
    "mkv_decode_plan_create": (c_int, [P, ctypes.POINTER(P)]),
    "mkv_decode_plan_destroy": (c_int, [P]),
    "mkv_decode_plan_build": (c_int, [P, I32P, i32, i32, P]),
    "mkv_decode_plan_info": (c_int, [P, I32P, I32P, I32P]),
    "mkv_decode_attention_planned": (c_int, [P, P, i32, P, P, P, P, f32, u32, P]),
    "mkv_decode_step": (c_int, [P, P, i32, P, P, P, P, P, P, f32, u32, P]),
    "mkv_decode_step_gather": (c_int, [P, P, i32, P, P, P, P, P, P, P, P, i64, f32, u32, P]),
    "mkv_decode_plan_build_suffixes": (c_int, [P, I32P, i32, i32, P]),
    "mkv_decode_step_shared_prefix": (c_int, [P, P, i32, P, P, P, P, P, i32, P, P, f32, u32, P]),
    "mkv_extend_attention": (c_int, [P, i32, P, P, P, P, P, P, i32, i32, i32, f32, u32, P]),
    "mkv_qk_norm_rope_append": (c_int, [P, i32, P, P, P, P, P, P, i32, f32, P, P, i32, P, u32, P]),
    "mkv_wire_export": (c_int, [P, P, i32, i32, i32, P, P, P]),
    "mkv_wire_import": (c_int, [P, P, i32, i32, i32, P, P, P, P]),
    "mkv_wire_header_init": (c_int, [DESC_P, i32, i32, i32, i64, WIRE_P]),
    "mkv_wire_header_check": (c_int, [DESC_P, WIRE_P]),
    "mkv_append_host": (c_int, [P, i32, P, P, U32P, i32, P]),
    "mkv_append_all_layers_host": (c_int, [P, P, P, U32P, i32, P]),
    "mkv_gather_host": (c_int, [P, i32, U32P, U32P, I32P, i32, P, P, i64, P]),
    "mkv_copy_blocks_host": (c_int, [P, U32P, U32P, i32, P]),
    "mkv_extend_attention_host": (c_int, [P, i32, P, P, I32P, I32P, U32P, U32P, i32, f32, u32, P]),
    "mkv_qk_norm_rope_append_host": (c_int, [P, i32, P, P, P, P, P, P, i32, f32, I32P, U32P, i32, P, u32, P]),
    "mkv_wire_export_host": (c_int, [P, U32P, i32, i32, i32, P, P, P]),
    "mkv_wire_import_host": (c_int, [P, U32P, i32, i32, i32, P, P, P, P]),
    "mkv_decode_plan_build_tables": (c_int, [P, I32P, U32P, U32P, i32, i32, P]),
    "mkv_decode_plan_build_shared_prefix": (c_int, [P, U32P, i32, I32P, U32P, U32P, i32, i32, P]),
    "mkv_validate_slots": (c_int, [DESC_P, I32P, i32]),
    "mkv_validate_block_tables": (c_int, [DESC_P, I32P, I32P, I32P, i32, i32]),
    "mkv_validate_copy_pairs": (c_int, [DESC_P, I32P, I32P, i32]),
    "mkv_buffer_alloc": (c_int, [c_int, u64, ctypes.POINTER(P)]),
    "mkv_buffer_free": (c_int, [P]),
    "mkv_memcpy_h2d": (c_int, [P, P, u64, P]),
    "mkv_memcpy_d2h": (c_int, [P, P, u64, P]),
    "mkv_stream_synchronize": (c_int, [P]),
    "mkv_last_error": (ctypes.c_char_p, []),
    "mkv_version": (c_int, []),
}

_device = None
_host = None


def _load(path: str, signatures: dict):
    if not os.path.exists(path):
        raise MkvLibraryMissing(
            f"{os.path.basename(path)} is not built; run `python -m mitten_amd._build` "
            "or __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    for name, (res, args) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def device_lib():
    """The HIP library. torch (if installed) is imported first so that both
    share the HIP runtime loaded from torch's lib directory."""
    global _device
    if _device is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        _device = _load(_build.DEVICE_LIB, DEVICE_SIGNATURES)
    return _device


def host_lib():
    global _host
    if _host is None:
        from ._host_sigs import HOST_SIGNATURES

        _host = _load(_build.HOST_LIB, HOST_SIGNATURES)
    return _host
