"""Device KV pool: the inference backend's device-buffer type, in Python.

`DeviceKvPool` owns one libmitten_kv pool (HBM, layout
[num_layers][2][num_blocks][page_size][num_kv_heads][head_dim]) and exposes the
four hot-path operations on torch device tensors:

    append(layer, k, v, slot_mapping)              model.rs:390-392 (Tensor::cat)
    gather(layer, block_indptr, block_ids, ctx_indptr, max_ctx_len)
                                                   design/phase0-deliverable.md:278
    copy_blocks(src, dst)                          (COW / compaction; no reference
                                                    counterpart)
    decode_attention(layer, q, block_indptr, block_ids, ctx_lens, max_ctx_len)
                                                   model.rs:394-416

torch is used only for device memory and streams; every operation runs in
the HIP library. Errors map onto the engine's error type
(inference-backend/src/error.rs:3-13): pool exhaustion -> OutOfKvPages,
everything else -> BackendError.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib

MKV_OK = 0
MKV_ERR_INVALID_ARGUMENT = 1
MKV_ERR_OUT_OF_MEMORY = 2
MKV_ERR_HIP = 3
MKV_ERR_DEVICE_INDEX = 4
MKV_ERR_NO_DEVICE = 5

DEVERR_SLOT, DEVERR_BLOCK, DEVERR_TABLE, DEVERR_COPY, DEVERR_CTX, DEVERR_CHECKSUM = 1, 2, 4, 8, 16, 32

ATTN_ZERO_SINK, ATTN_FORCE_VALU, ATTN_FORCE_MFMA, ATTN_PER_HEAD_LOADS, ATTN_CACHED_LOADS = 1, 2, 4, 8, 16
PREP_PLAIN_Q, PREP_NO_NORM = 1, 2

DTYPES = {"f32": 0, "bf16": 1}
PAGE_SIZE = 16


class EngineError(RuntimeError):
    """Mirror of inference-backend/src/error.rs EngineError."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class OutOfKvPages(EngineError):
    """EngineError::OutOfKvPages (error.rs:7-8)."""


class BackendError(EngineError):
    """EngineError::Backend(String) (error.rs:5-6)."""


class DeviceIndexError(BackendError):
    """A kernel met an out-of-range slot/block id (skipped, never dereferenced)."""

    def __init__(self, status: int, message: str, bits: int):
        super().__init__(status, message)
        self.bits = bits


def _raise(status: int) -> None:
    if status == MKV_OK:
        return
    msg = (_lib.device_lib().mkv_last_error() or b"").decode(errors="replace")
    if status == MKV_ERR_OUT_OF_MEMORY:
        raise OutOfKvPages(status, msg)
    raise BackendError(status, msg)


@dataclass(frozen=True)
class PoolDesc:
    """Pool geometry: the engine's ModelConfig (num_layers, num_kv_heads,
    head_dim; inference-backend/src/config.rs:1-11) plus num_q_heads and the
    EngineConfig pool size (num_kv_pages, page_size; inference-engine/src/config.rs:3-17)."""

    num_layers: int
    num_kv_heads: int
    num_q_heads: int
    head_dim: int
    num_blocks: int
    dtype: str = "bf16"
    page_size: int = PAGE_SIZE

    def c(self) -> _lib.PoolDescC:
        return _lib.PoolDescC(self.num_layers, self.num_kv_heads, self.num_q_heads, self.head_dim,
                              self.page_size, DTYPES[self.dtype], self.num_blocks)

    @property
    def elem_bytes(self) -> int:
        return 4 if self.dtype == "f32" else 2

    @property
    def block_bytes(self) -> int:
        """Bytes of one block of one layer, K or V."""
        return self.page_size * self.num_kv_heads * self.head_dim * self.elem_bytes

    @property
    def shape(self):
        return (self.num_layers, 2, self.num_blocks, self.page_size, self.num_kv_heads, self.head_dim)


def rope_inv_freq(rotary_dim: int, theta: float) -> np.ndarray:
    """The reference's RoPE frequency table, f32 throughout:
    1 / (theta as f32)^(2i / rotary_dim) for i < rotary_dim / 2
    (inference-model-qwen/src/model.rs:512-514)."""
    i = np.arange(rotary_dim // 2, dtype=np.float32)
    expo = (np.float32(2.0) * i) / np.float32(rotary_dim)
    return (np.float32(1.0) / np.power(np.float32(theta), expo)).astype(np.float32)


def required_bytes(desc: PoolDesc) -> int:
    """KvCachePool::required_bytes (inference-engine/src/kv_pool.rs:58-68)."""
    out = ctypes.c_uint64()
    _raise(_lib.device_lib().mkv_pool_required_bytes(ctypes.byref(desc.c()), ctypes.byref(out)))
    return out.value


def _i32p(a: np.ndarray):
    return a.ctypes.data_as(_lib.I32P)


def _u32p(a: np.ndarray):
    return a.ctypes.data_as(_lib.U32P)


def _is_host(x) -> bool:
    """Host metadata (numpy array, list, or a CPU tensor): goes through the
    *_host entry points, which validate and copy it before returning."""
    if isinstance(x, (np.ndarray, list, tuple)):
        return True
    try:
        import torch
    except ImportError:
        return False
    return isinstance(x, torch.Tensor) and not x.is_cuda


def _host_u32(x, name: str) -> np.ndarray:
    """Engine page ids / slots (u32). Values outside [0, 2^32) cannot be u32
    ids; they are refused here rather than wrapped by the cast (2^32 + 5
    would otherwise become id 5, a valid block of another sequence)."""
    a = np.asarray(x.numpy() if hasattr(x, "numpy") else x)
    if a.size:
        if a.dtype.kind not in "iu":
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} must hold integers, not {a.dtype}")
        if a.dtype.kind == "i" and int(a.min()) < 0:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} holds a negative id")
        if int(a.max()) > 0xFFFFFFFF:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} holds an id of 2^32 or more")
    return np.ascontiguousarray(a, np.uint32).reshape(-1)


def _host_i32(x, name: str = "lengths") -> np.ndarray:
    """Lengths, positions and the i32 metadata of the validators. Values
    outside i32 are refused rather than wrapped by the cast (a context of
    2^32 + 5 tokens would otherwise pass as 5)."""
    a = np.asarray(x.numpy() if hasattr(x, "numpy") else x)
    if a.size:
        if a.dtype.kind not in "iu":
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} must hold integers, not {a.dtype}")
        if int(a.max()) > 0x7FFFFFFF or (a.dtype.kind == "i" and int(a.min()) < -0x80000000):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} holds a value outside int32")
    return np.ascontiguousarray(a, np.int32).reshape(-1)


def validate_slots(desc: PoolDesc, slots) -> None:
    s = _host_i32(slots, "slots")
    _raise(_lib.device_lib().mkv_validate_slots(ctypes.byref(desc.c()), _i32p(s), s.size))


def validate_block_tables(desc: PoolDesc, indptr, ids, ctx_lens, max_ctx_len: int) -> None:
    ip = _host_i32(indptr, "indptr")
    ix = _host_i32(ids, "ids")
    cl = None if ctx_lens is None else _host_i32(ctx_lens, "ctx_lens")
    _raise(_lib.device_lib().mkv_validate_block_tables(
        ctypes.byref(desc.c()), _i32p(ip), _i32p(ix) if ix.size else None,
        _i32p(cl) if cl is not None else None, ip.size - 1, max_ctx_len))


def validate_copy_pairs(desc: PoolDesc, src, dst) -> None:
    s = _host_i32(src, "src")
    d = _host_i32(dst, "dst")
    if s.size != d.size:
        raise BackendError(MKV_ERR_INVALID_ARGUMENT, "src and dst differ in length")
    _raise(_lib.device_lib().mkv_validate_copy_pairs(ctypes.byref(desc.c()), _i32p(s), _i32p(d), s.size))


def _torch():
    import torch

    return torch


def _stream_handle(stream) -> ctypes.c_void_p:
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _tptr(t) -> ctypes.c_void_p:
    """Device pointer of an optional tensor (NULL for None)."""
    return ctypes.c_void_p(0) if t is None else ctypes.c_void_p(t.data_ptr())


class DeviceKvPool:
    """The device KV pool (design's KvBufferHandle, design/phase0-deliverable.md:1320-1332)."""

    def __init__(self, desc: PoolDesc, device: int = 0):
        self.desc = desc
        self.device = device
        self._lib = _lib.device_lib()
        h = ctypes.c_void_p()
        _raise(self._lib.mkv_pool_create(ctypes.byref(desc.c()), device, ctypes.byref(h)))
        self._h = h
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_uint64()
        _raise(self._lib.mkv_pool_buffer(self._h, ctypes.byref(ptr), ctypes.byref(nbytes)))
        self.data_ptr = ptr.value
        self.nbytes = nbytes.value

    # -- lifecycle -------------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.mkv_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def torch_dtype(self):
        torch = _torch()
        return torch.float32 if self.desc.dtype == "f32" else torch.bfloat16

    def _check_tensor(self, t, shape, name, dtype=None):
        torch = _torch()
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} must be a device tensor")
        want = dtype or self.torch_dtype
        if t.dtype != want:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} has dtype {t.dtype}, expected {want}")
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        if not t.is_contiguous():
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, f"{name} must be contiguous")

    def _i32(self, t, name, n=None):
        torch = _torch()
        self._check_tensor(t, (n,) if n is not None else None, name, dtype=torch.int32)

    # -- error word ---------------------------------------------------------------------
    def check(self, stream=None) -> None:
        """Synchronise and raise DeviceIndexError if a kernel met a bad id."""
        bits = ctypes.c_uint32()
        st = self._lib.mkv_pool_check(self._h, _stream_handle(stream), ctypes.byref(bits))
        if st == MKV_ERR_DEVICE_INDEX:
            raise DeviceIndexError(st, self._lib.mkv_last_error().decode(), bits.value)
        _raise(st)

    def set_launch_events(self, start, end) -> None:
        """Measurement: record `start` and `end` (HIP events: an object with a
        `handle`, a torch.cuda.Event already recorded once, or a raw handle)
        right before and after the attention kernel of the next decode call on
        this pool, before its merge (mkv_pool_set_launch_events). None, None
        forgets them."""

        def raw(ev):
            if ev is None:
                return None
            if hasattr(ev, "handle"):
                return ev.handle
            if hasattr(ev, "cuda_event"):
                return ctypes.c_void_p(ev.cuda_event)
            return ctypes.c_void_p(int(ev))

        _raise(self._lib.mkv_pool_set_launch_events(self._h, raw(start), raw(end)))

    # -- operations -----------------------------------------------------------------------
    def append(self, layer: int, k, v, slot_mapping, stream=None) -> None:
        """slot_mapping: device int32 tensor, or host u32 slots (numpy/list:
        mkv_append_host validates and copies them)."""
        d = self.desc
        host = _is_host(slot_mapping)
        sm = _host_u32(slot_mapping, "slot_mapping") if host else slot_mapping
        n = sm.shape[0]
        if not host:
            self._i32(sm, "slot_mapping", n)
        self._check_tensor(k, (n, d.num_kv_heads, d.head_dim), "k")
        self._check_tensor(v, (n, d.num_kv_heads, d.head_dim), "v")
        if host:
            _raise(self._lib.mkv_append_host(self._h, layer, _dptr(k), _dptr(v), _u32p(sm), n,
                                             _stream_handle(stream)))
        else:
            _raise(self._lib.mkv_append(self._h, layer, _dptr(k), _dptr(v), _dptr(sm), n,
                                        _stream_handle(stream)))

    def append_all_layers(self, k, v, slot_mapping, stream=None) -> None:
        d = self.desc
        host = _is_host(slot_mapping)
        sm = _host_u32(slot_mapping, "slot_mapping") if host else slot_mapping
        n = sm.shape[0]
        if not host:
            self._i32(sm, "slot_mapping", n)
        self._check_tensor(k, (d.num_layers, n, d.num_kv_heads, d.head_dim), "k")
        self._check_tensor(v, (d.num_layers, n, d.num_kv_heads, d.head_dim), "v")
        if host:
            _raise(self._lib.mkv_append_all_layers_host(self._h, _dptr(k), _dptr(v), _u32p(sm), n,
                                                        _stream_handle(stream)))
        else:
            _raise(self._lib.mkv_append_all_layers(self._h, _dptr(k), _dptr(v), _dptr(sm), n,
                                                   _stream_handle(stream)))

    def gather(self, layer: int, block_indptr, block_ids, ctx_indptr, max_ctx_len: int,
               out_k=None, out_v=None, total_tokens: int | None = None, stream=None):
        """Returns (k, v), each flat [sum(ctx) * Hkv * D]: sequence b occupies
        [Hkv][ctx_b][D] starting at element ctx_indptr[b]*Hkv*D."""
        torch = _torch()
        d = self.desc
        B = ctx_indptr.shape[0] - 1
        self._i32(block_indptr, "block_indptr", B + 1)
        self._i32(block_ids, "block_ids")
        self._i32(ctx_indptr, "ctx_indptr", B + 1)
        if total_tokens is None:
            total_tokens = int(ctx_indptr[-1].item())
        n = total_tokens * d.num_kv_heads * d.head_dim
        if out_k is None:
            out_k = torch.empty(n, dtype=self.torch_dtype, device=ctx_indptr.device)
        if out_v is None:
            out_v = torch.empty(n, dtype=self.torch_dtype, device=ctx_indptr.device)
        self._check_tensor(out_k, None, "out_k")
        self._check_tensor(out_v, None, "out_v")
        if out_k.numel() < n or out_v.numel() < n:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "gather outputs too small")
        row = d.num_kv_heads * d.head_dim
        cap = min(out_k.numel(), out_v.numel()) // row
        _raise(self._lib.mkv_gather(self._h, layer, _dptr(block_indptr), _dptr(block_ids),
                                    _dptr(ctx_indptr), B, max_ctx_len, _dptr(out_k), _dptr(out_v),
                                    cap, _stream_handle(stream)))
        return out_k, out_v

    def gather_host(self, layer: int, block_indptr, block_ids, ctx_lens, out_k=None, out_v=None, stream=None):
        """gather with host tables (u32 CSR) and host context lengths
        (mkv_gather_host). Returns (k, v) flat, as gather()."""
        torch = _torch()
        d = self.desc
        ip, ix = _host_u32(block_indptr, "block_indptr"), _host_u32(block_ids, "block_ids")
        cl = _host_i32(ctx_lens, "ctx_lens")
        B = cl.size
        if ip.size != B + 1:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "block_indptr must have num_seqs + 1 entries")
        n = int(cl.astype(np.int64).sum()) * d.num_kv_heads * d.head_dim
        dev = torch.device(f"cuda:{self.device}")
        if out_k is None:
            out_k = torch.empty(max(n, 1), dtype=self.torch_dtype, device=dev)
        if out_v is None:
            out_v = torch.empty(max(n, 1), dtype=self.torch_dtype, device=dev)
        self._check_tensor(out_k, None, "out_k")
        self._check_tensor(out_v, None, "out_v")
        cap = min(out_k.numel(), out_v.numel()) // (d.num_kv_heads * d.head_dim)
        _raise(self._lib.mkv_gather_host(self._h, layer, _u32p(ip), _u32p(ix) if ix.size else None, _i32p(cl), B,
                                         _dptr(out_k), _dptr(out_v), cap, _stream_handle(stream)))
        return out_k, out_v

    def copy_blocks(self, src, dst, stream=None) -> None:
        """src, dst: device int32 tensors, or host u32 ids (mkv_copy_blocks_host,
        which also checks that the pairs do not overlap)."""
        if _is_host(src) or _is_host(dst):
            s_, d_ = _host_u32(src, "src"), _host_u32(dst, "dst")
            if s_.size != d_.size:
                raise BackendError(MKV_ERR_INVALID_ARGUMENT, "src and dst differ in length")
            _raise(self._lib.mkv_copy_blocks_host(self._h, _u32p(s_), _u32p(d_), s_.size, _stream_handle(stream)))
            return
        n = src.shape[0]
        self._i32(src, "src", n)
        self._i32(dst, "dst", n)
        _raise(self._lib.mkv_copy_blocks(self._h, _dptr(src), _dptr(dst), n, _stream_handle(stream)))

    def workspace_size(self, num_seqs: int, max_ctx_len: int, split_tokens: int = 0) -> int:
        out = ctypes.c_uint64()
        _raise(self._lib.mkv_decode_attention_workspace_size(self._h, num_seqs, max_ctx_len,
                                                             split_tokens, ctypes.byref(out)))
        return out.value

    def decode_attention(self, layer: int, q, block_indptr, block_ids, ctx_lens, max_ctx_len: int,
                         scale: float | None = None, zero_sink: bool = False, out=None,
                         split_tokens: int = 0, workspace=None, kernel: str | None = None,
                         stream=None):
        """q: [B, Hq, D] in the pool dtype. Returns o: [B, Hq, D]."""
        torch = _torch()
        d = self.desc
        B = q.shape[0]
        self._check_tensor(q, (B, d.num_q_heads, d.head_dim), "q")
        self._i32(block_indptr, "block_indptr", B + 1)
        self._i32(block_ids, "block_ids")
        self._i32(ctx_lens, "ctx_lens", B)
        if out is None:
            out = torch.empty_like(q)
        self._check_tensor(out, (B, d.num_q_heads, d.head_dim), "out")
        if scale is None:
            scale = float(np.float32(d.head_dim ** -0.5))
        flags = ATTN_ZERO_SINK if zero_sink else 0
        if kernel == "valu":
            flags |= ATTN_FORCE_VALU
        elif kernel == "mfma":
            flags |= ATTN_FORCE_MFMA
        elif kernel is not None:
            raise ValueError(f"unknown kernel {kernel!r}")
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            self._check_tensor(workspace, None, "workspace", dtype=workspace.dtype)
            ws_ptr, ws_bytes = _dptr(workspace), workspace.numel() * workspace.element_size()
        _raise(self._lib.mkv_decode_attention(
            self._h, layer, _dptr(q), _dptr(out), _dptr(block_indptr), _dptr(block_ids),
            _dptr(ctx_lens), B, max_ctx_len, scale, flags, split_tokens, ws_ptr, ws_bytes,
            _stream_handle(stream)))
        return out

    def decode_attention_static(self, layer: int, q, block_indptr, block_ids, ctx_lens, max_ctx_len: int,
                                scale: float | None = None, zero_sink: bool = False, out=None,
                                split_tokens: int = 0, kernel: str | None = None, stream=None):
        """decode_attention with its split-K partials in the library's static
        device scratch (mkv_decode_attention_static): nothing is allocated."""
        torch = _torch()
        d = self.desc
        B = q.shape[0]
        self._check_tensor(q, (B, d.num_q_heads, d.head_dim), "q")
        self._i32(block_indptr, "block_indptr", B + 1)
        self._i32(block_ids, "block_ids")
        self._i32(ctx_lens, "ctx_lens", B)
        if out is None:
            out = torch.empty_like(q)
        self._check_tensor(out, (B, d.num_q_heads, d.head_dim), "out")
        if scale is None:
            scale = float(np.float32(d.head_dim ** -0.5))
        flags = ATTN_ZERO_SINK if zero_sink else 0
        if kernel == "valu":
            flags |= ATTN_FORCE_VALU
        elif kernel == "mfma":
            flags |= ATTN_FORCE_MFMA
        elif kernel is not None:
            raise ValueError(f"unknown kernel {kernel!r}")
        _raise(self._lib.mkv_decode_attention_static(
            self._h, layer, _dptr(q), _dptr(out), _dptr(block_indptr), _dptr(block_ids), _dptr(ctx_lens), B,
            max_ctx_len, scale, flags, split_tokens, _stream_handle(stream)))
        return out

    # -- planned path -------------------------------------------------------------------------
    def extend_attention(self, layer: int, q, q_indptr, block_indptr, block_ids, ctx_lens,
                         max_q_len: int, max_ctx_len: int, out=None, scale: float | None = None,
                         zero_sink: bool = False, stream=None):
        """Causal attention of each sequence's newest tokens (chunked prefill):
        q, out: [q_indptr[-1], Hq, D]; sequence b's n_b = q_indptr[b+1] - q_indptr[b]
        queries sit at positions [ctx_b - n_b, ctx_b) and attend keys 0..p."""
        torch = _torch()
        d = self.desc
        B = q_indptr.shape[0] - 1
        self._i32(q_indptr, "q_indptr", B + 1)
        self._i32(block_indptr, "block_indptr", B + 1)
        self._i32(block_ids, "block_ids")
        self._i32(ctx_lens, "ctx_lens", B)
        T = q.shape[0]
        self._check_tensor(q, (T, d.num_q_heads, d.head_dim), "q")
        if out is None:
            out = torch.empty_like(q)
        self._check_tensor(out, (T, d.num_q_heads, d.head_dim), "out")
        if scale is None:
            scale = float(np.float32(d.head_dim ** -0.5))
        flags = ATTN_ZERO_SINK if zero_sink else 0
        _raise(self._lib.mkv_extend_attention(
            self._h, layer, _dptr(q), _dptr(out), _dptr(q_indptr), _dptr(block_indptr), _dptr(block_ids),
            _dptr(ctx_lens), B, max_q_len, max_ctx_len, scale, flags, _stream_handle(stream)))
        return out

    def extend_attention_host(self, layer: int, q, q_lens, ctx_lens, block_indptr, block_ids, out=None,
                              scale: float | None = None, zero_sink: bool = False, stream=None):
        """extend_attention with host metadata (mkv_extend_attention_host):
        sequence b's q_lens[b] query rows follow sequence b-1's in q."""
        torch = _torch()
        d = self.desc
        ql, cl = _host_i32(q_lens, "q_lens"), _host_i32(ctx_lens, "ctx_lens")
        ip, ix = _host_u32(block_indptr, "block_indptr"), _host_u32(block_ids, "block_ids")
        T = int(ql.astype(np.int64).sum())
        self._check_tensor(q, (T, d.num_q_heads, d.head_dim), "q")
        if out is None:
            out = torch.empty_like(q)
        self._check_tensor(out, (T, d.num_q_heads, d.head_dim), "out")
        if ql.size != cl.size or ip.size != cl.size + 1:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "q_lens, ctx_lens and block_indptr disagree on num_seqs")
        if scale is None:
            scale = float(np.float32(d.head_dim ** -0.5))
        flags = ATTN_ZERO_SINK if zero_sink else 0
        _raise(self._lib.mkv_extend_attention_host(
            self._h, layer, _dptr(q), _dptr(out), _i32p(ql), _i32p(cl), _u32p(ip), _u32p(ix) if ix.size else None,
            cl.size, scale, flags, _stream_handle(stream)))
        return out

    def qk_norm_rope_append(self, layer: int, q, k, v, positions, slot_mapping, q_norm_w=None,
                            k_norm_w=None, inv_freq=None, eps: float = 1e-6, gated: bool = True,
                            out=None, stream=None):
        """Fused pre-attention step of one layer (inference-model-qwen/src/model.rs:371-392):
        RMSNorm(1 + w) of the q and k heads, NeoX RoPE on the first 2*len(inv_freq)
        dims at `positions`, k and v appended at `slot_mapping`; returns the prepared
        q [n, Hq, D]. q is [n, Hq, 2, D] (q then gate) when `gated`, else [n, Hq, D].
        Weights None skips the norm; inv_freq None skips RoPE."""
        torch = _torch()
        d = self.desc
        host = _is_host(slot_mapping)
        if host != _is_host(positions):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "positions and slot_mapping must both be host or device")
        if host:
            slot_mapping, positions = _host_u32(slot_mapping, "slot_mapping"), _host_i32(positions, "positions")
        n = slot_mapping.shape[0]
        if host:
            if positions.size != n:
                raise BackendError(MKV_ERR_INVALID_ARGUMENT, "positions and slot_mapping differ in length")
        else:
            self._i32(slot_mapping, "slot_mapping", n)
            self._i32(positions, "positions", n)
        qshape = (n, d.num_q_heads, 2, d.head_dim) if gated else (n, d.num_q_heads, d.head_dim)
        self._check_tensor(q, qshape, "q")
        self._check_tensor(k, (n, d.num_kv_heads, d.head_dim), "k")
        self._check_tensor(v, (n, d.num_kv_heads, d.head_dim), "v")
        flags = 0 if gated else PREP_PLAIN_Q
        if (q_norm_w is None) != (k_norm_w is None):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "give both norm weights or neither")
        if q_norm_w is None:
            flags |= PREP_NO_NORM
        else:
            self._check_tensor(q_norm_w, (d.head_dim,), "q_norm_w", dtype=torch.float32)
            self._check_tensor(k_norm_w, (d.head_dim,), "k_norm_w", dtype=torch.float32)
        rd = 0
        if inv_freq is not None:
            self._check_tensor(inv_freq, None, "inv_freq", dtype=torch.float32)
            rd = 2 * inv_freq.shape[0]
        if out is None:
            out = torch.empty((n, d.num_q_heads, d.head_dim), dtype=self.torch_dtype, device=q.device)
        self._check_tensor(out, (n, d.num_q_heads, d.head_dim), "out")
        nul = ctypes.c_void_p(0)
        fn = self._lib.mkv_qk_norm_rope_append_host if host else self._lib.mkv_qk_norm_rope_append
        _raise(fn(
            self._h, layer, _dptr(q), _dptr(k), _dptr(v),
            nul if q_norm_w is None else _dptr(q_norm_w), nul if k_norm_w is None else _dptr(k_norm_w),
            nul if inv_freq is None else _dptr(inv_freq), rd, eps,
            _i32p(positions) if host else _dptr(positions), _u32p(slot_mapping) if host else _dptr(slot_mapping),
            n, _dptr(out), flags, _stream_handle(stream)))
        return out

    def wire_block_bytes(self, num_layers: int | None = None) -> int:
        """Payload bytes of one block carrying `num_layers` layers (all by default)."""
        nl = self.desc.num_layers if num_layers is None else num_layers
        return nl * self.desc.block_bytes * 2

    def wire_export(self, block_ids, layer_begin: int = 0, num_layers: int | None = None, payload=None,
                    checksums=None, stream=None):
        """Blocks -> (payload uint8 [n * block_bytes], checksums int64 [n]):
        layers [layer_begin, layer_begin + num_layers) of each block, K and V,
        block-major, with the per-block sum64 checksum (mkv_wire_export)."""
        torch = _torch()
        host = _is_host(block_ids)
        if host:
            block_ids = _host_u32(block_ids, "block_ids")
        n = block_ids.shape[0]
        nl = self.desc.num_layers - layer_begin if num_layers is None else num_layers
        if not host:
            self._i32(block_ids, "block_ids", n)
        dev = torch.device(f"cuda:{self.device}")
        nbytes = n * self.wire_block_bytes(nl)
        if payload is None:
            payload = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        if checksums is None:
            checksums = torch.empty(n, dtype=torch.int64, device=dev)
        self._check_tensor(payload, (nbytes,), "payload", dtype=torch.uint8)
        self._check_tensor(checksums, (n,), "checksums", dtype=torch.int64)
        if host:
            _raise(self._lib.mkv_wire_export_host(self._h, _u32p(block_ids), n, layer_begin, nl, _dptr(payload),
                                                  _dptr(checksums), _stream_handle(stream)))
        else:
            _raise(self._lib.mkv_wire_export(self._h, _dptr(block_ids), n, layer_begin, nl, _dptr(payload),
                                             _dptr(checksums), _stream_handle(stream)))
        return payload, checksums

    def wire_import(self, block_ids, payload, layer_begin: int = 0, num_layers: int | None = None,
                    expected=None, checksums=None, stream=None):
        """payload -> blocks `block_ids` (mkv_wire_import); returns the checksums
        of the payload as received. With `expected`, a mismatch is reported by
        check() as DeviceIndexError with DEVERR_CHECKSUM."""
        torch = _torch()
        host = _is_host(block_ids)
        if host:
            block_ids = _host_u32(block_ids, "block_ids")
        n = block_ids.shape[0]
        nl = self.desc.num_layers - layer_begin if num_layers is None else num_layers
        if not host:
            self._i32(block_ids, "block_ids", n)
        self._check_tensor(payload, (n * self.wire_block_bytes(nl),), "payload", dtype=torch.uint8)
        if expected is not None:
            self._check_tensor(expected, (n,), "expected", dtype=torch.int64)
        if checksums is None:
            checksums = torch.empty(n, dtype=torch.int64, device=payload.device)
        self._check_tensor(checksums, (n,), "checksums", dtype=torch.int64)
        fn = self._lib.mkv_wire_import_host if host else self._lib.mkv_wire_import
        _raise(fn(self._h, _u32p(block_ids) if host else _dptr(block_ids), n, layer_begin, nl, _dptr(payload),
                  ctypes.c_void_p(0) if expected is None else _dptr(expected),
                  _dptr(checksums), _stream_handle(stream)))
        return checksums

    def plan(self, ctx_lens, pieces: int = 0, stream=None, block_indptr=None, block_ids=None) -> "DecodePlan":
        """Work plan of one decode step from host context lengths (tokens
        attended per sequence, including the token appended this step). With
        the batch's host page tables (u32 CSR block_indptr / block_ids) the
        plan holds them (mkv_decode_plan_build_tables) and the step's calls
        pass no tables."""
        p = DecodePlan(self)
        p.build(ctx_lens, pieces, stream, block_indptr, block_ids)
        return p

    def plan_suffixes(self, suffix_lens, pieces: int = 0, stream=None) -> "DecodePlan":
        """Work plan of a step over a shared prefix, from the host suffix
        lengths (tokens after the prefix, the appended one included); for
        decode_step_shared_prefix."""
        p = DecodePlan(self, suffixes=True)
        p.build(suffix_lens, pieces, stream)
        return p

    def plan_shared_prefix(self, prefix_ids, suffix_lens, block_indptr, block_ids, pieces: int = 0,
                           stream=None) -> "DecodePlan":
        """plan_suffixes holding the host tables of the suffixes and the
        prefix's u32 block ids (mkv_decode_plan_build_shared_prefix)."""
        p = DecodePlan(self, suffixes=True)
        p.build(suffix_lens, pieces, stream, block_indptr, block_ids, prefix_ids)
        return p

    def decode_step_shared_prefix(self, layer: int, plan, k_new, v_new, q, prefix_ids, block_indptr, block_ids,
                                  out=None, scale: float | None = None, zero_sink: bool = False,
                                  kernel: str | None = None, stream=None):
        """decode_step over a prefix of whole blocks that every sequence of the
        plan shares (prefix_ids, int32 on the device) followed by each
        sequence's suffix table (block_indptr / block_ids). k_new / v_new:
        [B, Hkv, D] appended at suffix position suffix_len - 1, or both None."""
        d = self.desc
        if not getattr(plan, "suffixes", False):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "the plan must come from plan_suffixes")
        out, scale, flags = self._planned_args(plan, q, block_indptr, block_ids, out, scale, zero_sink, kernel)
        if prefix_ids is not None:
            self._i32(prefix_ids, "prefix_ids")
        elif not plan.has_prefix:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "no prefix ids: pass them, or plan with plan_shared_prefix")
        B = plan.num_seqs
        if (k_new is None) != (v_new is None):
            raise ValueError("give both k_new and v_new, or neither")
        if k_new is not None:
            self._check_tensor(k_new, (B, d.num_kv_heads, d.head_dim), "k_new")
            self._check_tensor(v_new, (B, d.num_kv_heads, d.head_dim), "v_new")
        _raise(self._lib.mkv_decode_step_shared_prefix(
            self._h, plan._h, layer, _dptr(k_new) if k_new is not None else None,
            _dptr(v_new) if v_new is not None else None, _dptr(q), _dptr(out), _tptr(prefix_ids),
            0 if prefix_ids is None else int(prefix_ids.shape[0]), _tptr(block_indptr), _tptr(block_ids), scale,
            flags, _stream_handle(stream)))
        return out

    def _planned_args(self, plan, q, block_indptr, block_ids, out, scale, zero_sink, kernel, cached_loads=False):
        d = self.desc
        if plan.pool is not self:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "plan belongs to another pool")
        B = plan.num_seqs
        self._check_tensor(q, (B, d.num_q_heads, d.head_dim), "q")
        if (block_indptr is None) != (block_ids is None):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "give both device table tensors, or neither")
        if block_indptr is None:
            if not plan.has_tables:
                raise BackendError(MKV_ERR_INVALID_ARGUMENT, "no tables: pass device tables, or plan with host tables")
        else:
            self._i32(block_indptr, "block_indptr", B + 1)
            self._i32(block_ids, "block_ids")
        torch = _torch()
        if out is None:
            out = torch.empty_like(q)
        self._check_tensor(out, (B, d.num_q_heads, d.head_dim), "out")
        if scale is None:
            scale = float(np.float32(d.head_dim ** -0.5))
        flags = ATTN_ZERO_SINK if zero_sink else 0
        if kernel == "valu":
            flags |= ATTN_FORCE_VALU
        elif kernel == "mfma":
            flags |= ATTN_FORCE_MFMA
        elif kernel == "mfma-per-head":
            flags |= ATTN_FORCE_MFMA | ATTN_PER_HEAD_LOADS
        elif kernel is not None:
            raise ValueError(f"unknown kernel {kernel!r}")
        if cached_loads:
            flags |= ATTN_CACHED_LOADS
        return out, scale, flags

    def decode_attention_planned(self, layer: int, plan, q, block_indptr, block_ids, out=None,
                                 scale: float | None = None, zero_sink: bool = False,
                                 kernel: str | None = None, stream=None, cached_loads: bool = False):
        """cached_loads: K/V loads through the caches (MKV_ATTN_CACHED_LOADS),
        for batches whose tables share blocks."""
        out, scale, flags = self._planned_args(plan, q, block_indptr, block_ids, out, scale, zero_sink, kernel,
                                               cached_loads)
        _raise(self._lib.mkv_decode_attention_planned(
            self._h, plan._h, layer, _dptr(q), _dptr(out), _tptr(block_indptr), _tptr(block_ids),
            scale, flags, _stream_handle(stream)))
        return out

    def decode_step(self, layer: int, plan, k_new, v_new, q, block_indptr, block_ids, out=None,
                    scale: float | None = None, zero_sink: bool = False, kernel: str | None = None,
                    stream=None, cached_loads: bool = False, gather_out=None):
        """Append k_new/v_new ([B, Hkv, D]) at position ctx-1 of every sequence,
        then attend over ctx tokens, in one launch (plus the split-K merge).
        gather_out: (k, v) flat device tensors that also receive the layer's
        block-table gather (mkv_decode_step_gather)."""
        d = self.desc
        out, scale, flags = self._planned_args(plan, q, block_indptr, block_ids, out, scale, zero_sink, kernel,
                                               cached_loads)
        B = plan.num_seqs
        self._check_tensor(k_new, (B, d.num_kv_heads, d.head_dim), "k_new")
        self._check_tensor(v_new, (B, d.num_kv_heads, d.head_dim), "v_new")
        if gather_out is None:
            _raise(self._lib.mkv_decode_step(
                self._h, plan._h, layer, _dptr(k_new), _dptr(v_new), _dptr(q), _dptr(out),
                _tptr(block_indptr), _tptr(block_ids), scale, flags, _stream_handle(stream)))
        else:
            gk, gv, cap = self._gather_outputs(gather_out)
            _raise(self._lib.mkv_decode_step_gather(
                self._h, plan._h, layer, _dptr(k_new), _dptr(v_new), _dptr(q), _dptr(out),
                _tptr(block_indptr), _tptr(block_ids), gk, gv, cap, scale, flags, _stream_handle(stream)))
        return out

    def _gather_outputs(self, gather_out):
        """(k, v) flat device tensors of the pool dtype -> (k ptr, v ptr, capacity in tokens)."""
        d = self.desc
        gk, gv = gather_out
        self._check_tensor(gk, None, "gather k")
        self._check_tensor(gv, None, "gather v")
        cap = min(gk.numel(), gv.numel()) // (d.num_kv_heads * d.head_dim)
        return _dptr(gk), _dptr(gv), cap

    def bind_decode_step(self, plan, k_new, v_new, q, block_indptr, block_ids, out,
                         scale: float | None = None, zero_sink: bool = False,
                         kernel: str | None = None, stream=None, cached_loads: bool = False,
                         gather_out=None):
        """Validates, once, the buffers of every layer of one decode step
        (k_new, v_new: [L, B, Hkv, D]; q, out: [L, B, Hq, D]) and returns
        `run(layer)`, which enqueues mkv_decode_step for that layer with no
        per-call Python checks (the engine's per-layer hot loop).
        gather_out: (k, v) flat device tensors that every layer's call also
        writes its block-table gather into (mkv_decode_step_gather)."""
        d = self.desc
        L, B = d.num_layers, plan.num_seqs
        self._check_tensor(k_new, (L, B, d.num_kv_heads, d.head_dim), "k_new")
        self._check_tensor(v_new, (L, B, d.num_kv_heads, d.head_dim), "v_new")
        self._check_tensor(q, (L, B, d.num_q_heads, d.head_dim), "q")
        self._check_tensor(out, (L, B, d.num_q_heads, d.head_dim), "out")
        _, scale, flags = self._planned_args(plan, q[0], block_indptr, block_ids, out[0], scale, zero_sink,
                                             kernel, cached_loads)
        fn = self._lib.mkv_decode_step if gather_out is None else self._lib.mkv_decode_step_gather
        gx = () if gather_out is None else self._gather_outputs(gather_out)
        h, ph = self._h, plan._h
        sh = _stream_handle(stream)
        kv_stride = B * d.num_kv_heads * d.head_dim * d.elem_bytes
        qo_stride = B * d.num_q_heads * d.head_dim * d.elem_bytes
        kb, vb, qb, ob = k_new.data_ptr(), v_new.data_ptr(), q.data_ptr(), out.data_ptr()
        ip, ix = _tptr(block_indptr), _tptr(block_ids)
        args = [(h, ph, layer, ctypes.c_void_p(kb + layer * kv_stride), ctypes.c_void_p(vb + layer * kv_stride),
                 ctypes.c_void_p(qb + layer * qo_stride), ctypes.c_void_p(ob + layer * qo_stride), ip, ix)
                + gx + (scale, flags, sh) for layer in range(L)]
        keep = (k_new, v_new, q, out, block_indptr, block_ids, gather_out)

        def run(layer: int) -> None:
            st = fn(*args[layer])
            if st:
                _raise(st)

        run.keep_alive = keep
        return run

    def bind_decode_step_shared_prefix(self, plan, k_new, v_new, q, prefix_ids, block_indptr, block_ids, out,
                                       scale: float | None = None, zero_sink: bool = False, stream=None):
        """bind_decode_step for decode_step_shared_prefix: validates the
        buffers of every layer once ([L, B, ...]) and returns `run(layer)`."""
        d = self.desc
        if not getattr(plan, "suffixes", False):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "the plan must come from plan_suffixes")
        L, B = d.num_layers, plan.num_seqs
        self._check_tensor(k_new, (L, B, d.num_kv_heads, d.head_dim), "k_new")
        self._check_tensor(v_new, (L, B, d.num_kv_heads, d.head_dim), "v_new")
        self._check_tensor(q, (L, B, d.num_q_heads, d.head_dim), "q")
        self._check_tensor(out, (L, B, d.num_q_heads, d.head_dim), "out")
        if prefix_ids is not None:
            self._i32(prefix_ids, "prefix_ids")
        elif not plan.has_prefix:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "no prefix ids: pass them, or plan with plan_shared_prefix")
        _, scale, flags = self._planned_args(plan, q[0], block_indptr, block_ids, out[0], scale, zero_sink, None)
        fn = self._lib.mkv_decode_step_shared_prefix
        kv_stride = B * d.num_kv_heads * d.head_dim * d.elem_bytes
        qo_stride = B * d.num_q_heads * d.head_dim * d.elem_bytes
        kb, vb, qb, ob = k_new.data_ptr(), v_new.data_ptr(), q.data_ptr(), out.data_ptr()
        pre, npre = _tptr(prefix_ids), 0 if prefix_ids is None else int(prefix_ids.shape[0])
        ip, ix, sh = _tptr(block_indptr), _tptr(block_ids), _stream_handle(stream)
        args = [(self._h, plan._h, layer, ctypes.c_void_p(kb + layer * kv_stride),
                 ctypes.c_void_p(vb + layer * kv_stride), ctypes.c_void_p(qb + layer * qo_stride),
                 ctypes.c_void_p(ob + layer * qo_stride), pre, npre, ip, ix, scale, flags, sh) for layer in range(L)]
        keep = (k_new, v_new, q, out, prefix_ids, block_indptr, block_ids)

        def run(layer: int) -> None:
            st = fn(*args[layer])
            if st:
                _raise(st)

        run.keep_alive = keep
        return run

    # -- host read-back / upload (tests) ------------------------------------------------------
    def read(self) -> np.ndarray:
        """Copy of the whole pool as numpy (uint16 bit patterns for bf16)."""
        dt = np.float32 if self.desc.dtype == "f32" else np.uint16
        host = np.empty(self.desc.shape, dt)
        _raise(self._lib.mkv_memcpy_d2h(ctypes.c_void_p(host.ctypes.data), ctypes.c_void_p(self.data_ptr),
                                        self.nbytes, _stream_handle(None)))
        return host

    def write(self, host: np.ndarray) -> None:
        """Upload a whole-pool numpy array (same layout/bytes) and synchronise."""
        host = np.ascontiguousarray(host)
        if host.nbytes != self.nbytes:
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "host array size differs from the pool")
        s = _stream_handle(None)
        _raise(self._lib.mkv_memcpy_h2d(ctypes.c_void_p(self.data_ptr), ctypes.c_void_p(host.ctypes.data),
                                        self.nbytes, s))
        _raise(self._lib.mkv_stream_synchronize(s))

    def tensor(self):
        """Zero-copy torch view of the pool buffer, shape `desc.shape`."""
        torch = _torch()
        dt = self.torch_dtype

        class _View:
            pass

        view = _View()
        typestr = "<f4" if self.desc.dtype == "f32" else "<i2"
        view.__cuda_array_interface__ = {
            "shape": tuple(int(x) for x in self.desc.shape),
            "typestr": typestr,
            "data": (self.data_ptr, False),
            "version": 3,
            "strides": None,
        }
        t = torch.as_tensor(view, device=f"cuda:{self.device}")
        return t if self.desc.dtype == "f32" else t.view(dt)


class DecodePlan:
    """Host-built work plan of one decode step (balanced pieces of the batch's
    blocks), reused by every layer of the step."""

    def __init__(self, pool: DeviceKvPool, suffixes: bool = False):
        self.pool = pool
        self._lib = pool._lib
        self.suffixes = suffixes  # built over the suffixes of a shared prefix
        h = ctypes.c_void_p()
        _raise(self._lib.mkv_decode_plan_create(pool._h, ctypes.byref(h)))
        self._h = h
        self.num_seqs = 0
        self.has_tables = False
        self.has_prefix = False

    def build(self, ctx_lens, pieces: int = 0, stream=None, block_indptr=None, block_ids=None,
              prefix_ids=None) -> None:
        """ctx_lens: host lengths. block_indptr / block_ids: the batch's host
        page tables (u32 CSR), held by the plan; prefix_ids: a shared prefix's
        host block ids (suffix plans only). The library copies them before
        returning."""
        c = _host_i32(ctx_lens, "ctx_lens")
        sh = _stream_handle(stream)
        if (block_indptr is None) != (block_ids is None):
            raise BackendError(MKV_ERR_INVALID_ARGUMENT, "give both block_indptr and block_ids, or neither")
        if block_indptr is None:
            if prefix_ids is not None:
                raise BackendError(MKV_ERR_INVALID_ARGUMENT, "prefix ids need the suffix tables")
            fn = self._lib.mkv_decode_plan_build_suffixes if self.suffixes else self._lib.mkv_decode_plan_build
            _raise(fn(self._h, _i32p(c), c.size, pieces, sh))
        else:
            ip, ix = _host_u32(block_indptr, "block_indptr"), _host_u32(block_ids, "block_ids")
            if ip.size != c.size + 1:
                raise BackendError(MKV_ERR_INVALID_ARGUMENT, "block_indptr must have num_seqs + 1 entries")
            ixp = _u32p(ix) if ix.size else None
            if self.suffixes:
                if prefix_ids is None:
                    raise BackendError(MKV_ERR_INVALID_ARGUMENT, "a suffix plan with tables needs the prefix ids")
                pre = _host_u32(prefix_ids, "prefix_ids")
                _raise(self._lib.mkv_decode_plan_build_shared_prefix(
                    self._h, _u32p(pre), pre.size, _i32p(c), _u32p(ip), ixp, c.size, pieces, sh))
            else:
                if prefix_ids is not None:
                    raise BackendError(MKV_ERR_INVALID_ARGUMENT, "prefix ids belong to a suffix plan")
                _raise(self._lib.mkv_decode_plan_build_tables(self._h, _i32p(c), _u32p(ip), ixp, c.size, pieces,
                                                              sh))
        self.num_seqs = int(c.size)
        self.has_tables = block_indptr is not None
        self.has_prefix = prefix_ids is not None

    def info(self):
        p, bp, m = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        _raise(self._lib.mkv_decode_plan_info(self._h, ctypes.byref(p), ctypes.byref(bp), ctypes.byref(m)))
        return {"pieces": p.value, "blocks_per_piece": bp.value, "merge_seqs": m.value}

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.mkv_decode_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
