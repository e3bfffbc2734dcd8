"""KV blocks as bytes: the wire / disk form of `mkv_wire_export` and
`mkv_wire_import` (include/mitten_kv.h), for offload to host memory or disk
and for handing a request's pages to another pool.

A message is: a 64-byte `mkv_wire_header` | one u64 checksum per block |
zero padding | the payload at `header.payload_offset` (a multiple of 4096),
[num_blocks][num_layers][K, V][page_size][num_kv_heads][head_dim] in the
pool dtype. It is the byte form of the reference's KvHandoff
(design/phase2b-deliverable.md:272-289: request pages + cached_len) and of
its per-layer KV offload files (design/phase1-deliverable.md:253-339).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .device_pool import MKV_ERR_INVALID_ARGUMENT, BackendError, DeviceKvPool, _host_i32, _raise

HEADER_BYTES = 64


@dataclass
class WireMessage:
    header: _lib.WireHeaderC
    checksums: np.ndarray   # int64 [num_blocks] (u64 bit patterns)
    payload: "object"       # torch uint8 tensor (device or host)


def header(pool: DeviceKvPool, num_blocks: int, cached_len: int, layer_begin: int = 0,
           num_layers: int | None = None) -> _lib.WireHeaderC:
    nl = pool.desc.num_layers - layer_begin if num_layers is None else num_layers
    h = _lib.WireHeaderC()
    _raise(_lib.device_lib().mkv_wire_header_init(ctypes.byref(pool.desc.c()), layer_begin, nl, num_blocks,
                                                  cached_len, ctypes.byref(h)))
    return h


def check_header(pool: DeviceKvPool, h: _lib.WireHeaderC) -> None:
    _raise(_lib.device_lib().mkv_wire_header_check(ctypes.byref(pool.desc.c()), ctypes.byref(h)))


def encode(h: _lib.WireHeaderC, checksums: np.ndarray, payload: bytes | memoryview) -> bytes:
    """The message bytes: header, checksums, padding, payload."""
    sums = np.ascontiguousarray(checksums, np.int64).astype("<i8")
    if sums.size != h.num_blocks or len(payload) != h.num_blocks * h.block_bytes:
        raise BackendError(MKV_ERR_INVALID_ARGUMENT, "checksums or payload do not match the header")
    head = bytes(h) + sums.tobytes()
    return head + bytes(h.payload_offset - len(head)) + bytes(payload)


def decode(buf: bytes | memoryview) -> tuple[_lib.WireHeaderC, np.ndarray, memoryview]:
    """Split a message into (header, checksums, payload view); checks sizes only."""
    mv = memoryview(buf)
    if len(mv) < HEADER_BYTES:
        raise BackendError(MKV_ERR_INVALID_ARGUMENT, "message shorter than its header")
    h = _lib.WireHeaderC.from_buffer_copy(mv[:HEADER_BYTES])
    end_sums = HEADER_BYTES + 8 * h.num_blocks
    need = h.payload_offset + h.num_blocks * h.block_bytes
    if h.num_blocks < 0 or h.payload_offset < end_sums or len(mv) != need:
        raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"message of {len(mv)} bytes, header says {need}")
    sums = np.frombuffer(mv[HEADER_BYTES:end_sums], dtype="<i8").astype(np.int64)
    return h, sums, mv[h.payload_offset:need]


def export_blocks(pool: DeviceKvPool, block_ids, cached_len: int, layer_begin: int = 0,
                  num_layers: int | None = None, stream=None) -> bytes:
    """Device blocks -> message bytes (synchronises `stream`)."""
    import torch

    ids = _ids(block_ids)
    h = header(pool, ids.shape[0], cached_len, layer_begin, num_layers)
    payload, sums = pool.wire_export(ids, layer_begin, h.num_layers, stream=stream)
    (stream or torch.cuda.current_stream()).synchronize()
    pool.check(stream)
    return encode(h, sums.cpu().numpy(), payload.cpu().numpy().tobytes())


def import_blocks(pool: DeviceKvPool, message: bytes | memoryview, block_ids, stream=None) -> _lib.WireHeaderC:
    """Message bytes -> device blocks `block_ids` (fresh, distinct), verifying
    every block's checksum; raises DeviceIndexError (DEVERR_CHECKSUM) on a
    mismatch, BackendError on a header this pool cannot take."""
    import torch

    h, sums, payload = decode(message)
    check_header(pool, h)
    ids = _ids(block_ids)
    if ids.shape[0] != h.num_blocks:
        raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{h.num_blocks} blocks in the message, "
                                                     f"{ids.shape[0]} destinations given")
    dev = ids.device
    host = torch.frombuffer(bytearray(payload), dtype=torch.uint8) if h.num_blocks else \
        torch.empty(0, dtype=torch.uint8)
    d_payload = host.to(dev)
    expected = torch.from_numpy(sums.copy()).to(dev)
    pool.wire_import(ids, d_payload, h.layer_begin, h.num_layers, expected=expected, stream=stream)
    pool.check(stream)
    return h


def _ids(block_ids):
    import torch

    if isinstance(block_ids, torch.Tensor):
        return block_ids
    return torch.from_numpy(_host_i32(block_ids, "block_ids")).cuda()
