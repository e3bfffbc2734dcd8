"""ctypes front-end of the CPU oracle (oracle/mkv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
bench.py's CPU-baseline leg, always as the checker or the timed CPU baseline,
never as the product path.  The HIP library (mitten_amd) does not import this.

Arrays are numpy; bf16 data is carried as ``np.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libmkv_oracle.so")

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", HERE, "-B" if force else "-s"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


class PoolDesc(ctypes.Structure):
    _fields_ = [
        ("num_layers", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int64),
        ("elem_bytes", ctypes.c_int32),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, f32, f64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        dp = ctypes.POINTER(PoolDesc)
        sig = {
            "orc_splitmix64": (ctypes.c_uint64, [P]),
            "orc_fill_normal_f32": (None, [ctypes.c_uint64, i64, P]),
            "orc_bounded": (ctypes.c_uint32, [P, ctypes.c_uint32]),
            "orc_f32_to_bf16": (None, [P, P, i64]),
            "orc_bf16_to_f32": (None, [P, P, i64]),
            "orc_pool_bytes": (i64, [dp]),
            "orc_append": (i64, [dp, P, ctypes.c_int, P, P, P, i64]),
            "orc_gather": (ctypes.c_int, [dp, P, ctypes.c_int, P, P, P, i32, P, P]),
            "orc_copy_blocks": (ctypes.c_int, [dp, P, P, P, i64]),
            "orc_norm_rope_rows": (None, [P, i64, i32, P, f32, P, i32, P]),
            "orc_wire_checksums": (None, [P, i64, i64, P]),
            "orc_wire_export": (i64, [dp, P, P, i64, ctypes.c_int, ctypes.c_int, P, P]),
            "orc_wire_import": (i64, [dp, P, P, i64, ctypes.c_int, ctypes.c_int, P, P]),
            "orc_decode_attention_f32": (ctypes.c_int, [dp, P, ctypes.c_int, P, i32, i32, P, P, P,
                                                        f32, ctypes.c_int, P]),
            "orc_decode_attention_f64": (ctypes.c_int, [dp, P, ctypes.c_int, P, i32, i32, P, P, P,
                                                        f64, ctypes.c_int, P]),
            "orc_ref_faithful_decode": (ctypes.c_int, [P, P, i64, i32, i32, i32, P, P, P, f32, P]),
            "orc_ref_faithful_batch": (ctypes.c_double, [P, i32, i32, i32, i32, ctypes.c_uint64]),
            "orc_ref_faithful_decode_copy": (ctypes.c_int, [P, P, i64, i32, i32, i32, P, P, P, f32, P]),
            "orc_num_threads": (ctypes.c_int, []),
            "orc_set_num_threads": (None, [ctypes.c_int]),
            "orc_set_setup_threads": (None, [ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


# ---------------------------------------------------------------- data ----

def fill_normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(ctypes.c_uint64(seed), n, _p(out))
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32(_p(x), _p(out), x.size)
    return out


class SplitMix64:
    """Seeded integer stream shared with the C oracle (SplitMix64 + Lemire)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed)

    def next(self) -> int:
        return lib().orc_splitmix64(ctypes.byref(self.state))

    def bounded(self, n: int) -> int:
        return lib().orc_bounded(ctypes.byref(self.state), n)

    def uniform_int(self, lo: int, hi: int) -> int:
        """Uniform integer in [lo, hi]."""
        return lo + self.bounded(hi - lo + 1)


# ---------------------------------------------------------------- pool ----

def desc(num_layers, num_kv_heads, head_dim, num_blocks, elem_bytes, page_size=16) -> PoolDesc:
    return PoolDesc(num_layers, num_kv_heads, head_dim, page_size, num_blocks, elem_bytes)


def pool_bytes(d: PoolDesc) -> int:
    return lib().orc_pool_bytes(ctypes.byref(d))


def pool_shape(d: PoolDesc):
    return (d.num_layers, 2, d.num_blocks, d.page_size, d.num_kv_heads, d.head_dim)


def append(d: PoolDesc, pool: np.ndarray, layer: int, k: np.ndarray, v: np.ndarray,
           slots: np.ndarray) -> int:
    """In-place append into ``pool``; returns -1 or the first bad token index."""
    slots = np.ascontiguousarray(slots, np.int32)
    return lib().orc_append(ctypes.byref(d), _p(pool), layer, _p(k), _p(v), _p(slots), slots.size)


def gather(d: PoolDesc, pool: np.ndarray, layer: int, indptr, indices, ctx_len):
    indptr = np.ascontiguousarray(indptr, np.int32)
    indices = np.ascontiguousarray(indices, np.int32)
    ctx_len = np.ascontiguousarray(ctx_len, np.int32)
    n = int(ctx_len.sum()) * d.num_kv_heads * d.head_dim
    dt = pool.dtype
    dk, dv = np.empty(n, dt), np.empty(n, dt)
    rc = lib().orc_gather(ctypes.byref(d), _p(pool), layer, _p(indptr), _p(indices), _p(ctx_len),
                          ctx_len.size, _p(dk), _p(dv))
    if rc != 0:
        raise ValueError("orc_gather: invalid block table or context length")
    return dk, dv


def copy_blocks(d: PoolDesc, pool: np.ndarray, src, dst) -> None:
    src = np.ascontiguousarray(src, np.int32)
    dst = np.ascontiguousarray(dst, np.int32)
    if lib().orc_copy_blocks(ctypes.byref(d), _p(pool), _p(src), _p(dst), src.size) != 0:
        raise ValueError("orc_copy_blocks: block id out of range")


def norm_rope_rows(x: np.ndarray, w, eps: float, inv_freq, pos) -> np.ndarray:
    """RMSNorm(1 + w) then partial NeoX RoPE of each row (model.rs:104-108,
    508-540); x: [..., D] f32 values, pos: one position per row of x[..., 0]
    (broadcast over the middle axes by the caller). w None skips the norm,
    inv_freq None (or empty) skips RoPE. Returns a new f32 array."""
    y = np.array(x, dtype=np.float32, order="C", copy=True)
    D = y.shape[-1]
    rows = y.size // D
    pos = np.ascontiguousarray(pos, np.int32).reshape(-1)
    if pos.size != rows:
        raise ValueError("one position per row")
    wv = None if w is None else np.ascontiguousarray(w, np.float32)
    f = np.zeros(0, np.float32) if inv_freq is None else np.ascontiguousarray(inv_freq, np.float32)
    lib().orc_norm_rope_rows(_p(y), rows, D, None if wv is None else _p(wv), float(np.float32(eps)),
                             _p(f) if f.size else None, 2 * f.size, _p(pos))
    return y


def qk_norm_rope_append(d: PoolDesc, pool: np.ndarray, layer: int, q: np.ndarray, k: np.ndarray,
                        v: np.ndarray, q_w, k_w, inv_freq, eps: float, positions, slots) -> np.ndarray:
    """The fused pre-attention step of GatedAttention::forward
    (inference-model-qwen/src/model.rs:371-392) on one layer: q [n, Hq, 2, D]
    (q then gate) or [n, Hq, D], k, v [n, Hkv, D] as f32 values; q and k heads
    are normed and rotated at their token's position, k (rounded to the pool
    dtype) and v are appended at `slots` in place; returns q in the pool
    dtype's storage (np.uint16 bf16 bits or f32)."""
    q = np.asarray(q, np.float32)
    if q.ndim == 4:
        q = q[:, :, 0, :]
    n, Hq, D = q.shape
    Hkv = k.shape[1]
    pos = np.asarray(positions, np.int32)
    qo = norm_rope_rows(q, q_w, eps, inv_freq, np.repeat(pos, Hq))
    ko = norm_rope_rows(np.asarray(k, np.float32), k_w, eps, inv_freq, np.repeat(pos, Hkv))
    if d.elem_bytes == 2:
        qo, ko, vs = f32_to_bf16(qo), f32_to_bf16(ko), f32_to_bf16(np.asarray(v, np.float32))
    else:
        vs = np.ascontiguousarray(v, np.float32)
    bad = append(d, pool, layer, np.ascontiguousarray(ko), np.ascontiguousarray(vs), slots)
    if bad >= 0:
        raise ValueError(f"slot of token {bad} outside the pool")
    return qo


def wire_checksums(payload: np.ndarray, n: int, block_bytes: int) -> np.ndarray:
    """sum64 of each block of a payload (include/mitten_kv.h), as int64 bit patterns."""
    p = np.ascontiguousarray(payload).view(np.uint8)
    out = np.empty(n, np.uint64)
    lib().orc_wire_checksums(_p(p), n, block_bytes, _p(out))
    return out.view(np.int64)


def wire_export(d: PoolDesc, pool: np.ndarray, ids, layer_begin: int, num_layers: int):
    """(payload uint8 [n * num_layers * 2 * block_bytes], checksums int64 [n])."""
    ids = np.ascontiguousarray(ids, np.int32)
    per = num_layers * 2 * d.page_size * d.num_kv_heads * d.head_dim * d.elem_bytes
    payload = np.empty(ids.size * per, np.uint8)
    sums = np.empty(ids.size, np.uint64)
    bad = lib().orc_wire_export(ctypes.byref(d), _p(pool), _p(ids), ids.size, layer_begin, num_layers,
                                _p(payload), _p(sums))
    if bad >= 0:
        raise ValueError(f"block id {ids[bad]} outside the pool")
    return payload, sums.view(np.int64)


def wire_import(d: PoolDesc, pool: np.ndarray, ids, layer_begin: int, num_layers: int,
                payload: np.ndarray) -> np.ndarray:
    """In-place scatter of a payload into blocks `ids`; returns its checksums."""
    ids = np.ascontiguousarray(ids, np.int32)
    p = np.ascontiguousarray(payload).view(np.uint8)
    sums = np.empty(ids.size, np.uint64)
    bad = lib().orc_wire_import(ctypes.byref(d), _p(pool), _p(ids), ids.size, layer_begin, num_layers,
                                _p(p), _p(sums))
    if bad >= 0:
        raise ValueError(f"block id {ids[bad]} outside the pool")
    return sums.view(np.int64)


def decode_attention(d: PoolDesc, pool: np.ndarray, layer: int, q: np.ndarray, indptr, indices,
                     ctx_len, scale: float | None = None, zero_sink: bool = False,
                     precision: str = "f32") -> np.ndarray:
    """q: [B, Hq, D] f32 values (bf16 queries passed already widened)."""
    q = np.ascontiguousarray(q, np.float32)
    B, Hq, D = q.shape
    indptr = np.ascontiguousarray(indptr, np.int32)
    indices = np.ascontiguousarray(indices, np.int32)
    ctx_len = np.ascontiguousarray(ctx_len, np.int32)
    if scale is None:
        scale = float(np.float32(D ** -0.5))
    if precision == "f32":
        o = np.empty((B, Hq, D), np.float32)
        rc = lib().orc_decode_attention_f32(ctypes.byref(d), _p(pool), layer, _p(q), B, Hq,
                                            _p(indptr), _p(indices), _p(ctx_len), scale,
                                            int(zero_sink), _p(o))
    else:
        o = np.empty((B, Hq, D), np.float64)
        rc = lib().orc_decode_attention_f64(ctypes.byref(d), _p(pool), layer, _p(q), B, Hq,
                                            _p(indptr), _p(indices), _p(ctx_len), float(scale),
                                            int(zero_sink), _p(o))
    if rc != 0:
        raise ValueError("orc_decode_attention: invalid arguments")
    return o


def extend_attention(d: PoolDesc, pool: np.ndarray, layer: int, q: np.ndarray, q_indptr, indptr, indices,
                     ctx_len, scale: float | None = None, zero_sink: bool = False,
                     precision: str = "f32") -> np.ndarray:
    """Causal attention of each sequence's newest tokens, the seq_q > 1 path of
    inference-model-qwen/src/model.rs:410-416 with the mask of model.rs:542-555:
    query i of sequence b sits at position p = ctx_b - n_b + i and attends keys
    0..p (the mask's -1e10 makes every later key's weight exactly 0 in f32).
    That is, each query is a decode query over the first p + 1 tokens of its
    sequence's table, which is how it is computed here (one virtual sequence
    per query token). q: [sum n_b, Hq, D] f32 values."""
    q_indptr = np.asarray(q_indptr, np.int64)
    indptr = np.asarray(indptr, np.int64)
    indices = np.asarray(indices, np.int32)
    ctx_len = np.asarray(ctx_len, np.int64)
    v_ptr, v_ids, v_ctx = [0], [], []
    for b in range(ctx_len.size):
        nb = int(q_indptr[b + 1] - q_indptr[b])
        table = indices[indptr[b]:indptr[b + 1]]
        for i in range(nb):
            p = int(ctx_len[b]) - nb + i
            need = p // d.page_size + 1
            v_ids.append(table[:need])
            v_ptr.append(v_ptr[-1] + need)
            v_ctx.append(p + 1)
    if not v_ctx:
        return np.empty((0,) + q.shape[1:], np.float32 if precision == "f32" else np.float64)
    return decode_attention(d, pool, layer, q, np.asarray(v_ptr, np.int32), np.concatenate(v_ids),
                            np.asarray(v_ctx, np.int32), scale=scale, zero_sink=zero_sink,
                            precision=precision)


def ref_faithful_batch(ctx, Hkv: int, Hq: int, D: int, seed: int = 1) -> float:
    """Seconds for one reference-faithful decode step (one layer) of every
    sequence; ctx[b] counts the appended token."""
    c = np.ascontiguousarray(ctx, np.int32)
    return lib().orc_ref_faithful_batch(_p(c), c.size, Hkv, Hq, D, ctypes.c_uint64(seed))


def ref_faithful_decode(kcache: np.ndarray, vcache: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
                        q: np.ndarray, scale: float | None = None) -> np.ndarray:
    """The timed CPU baseline's decode of one sequence (contiguous caches
    [Hkv, T, D] grown by a copy, repeat_kv materialised, mask, softmax, two
    matmuls: model.rs:390-416). Returns o [Hq, D]."""
    kc, vc = np.ascontiguousarray(kcache, np.float32), np.ascontiguousarray(vcache, np.float32)
    Hkv, T, D = kc.shape
    q = np.ascontiguousarray(q, np.float32)
    Hq = q.shape[0]
    kn, vn = np.ascontiguousarray(k_new, np.float32), np.ascontiguousarray(v_new, np.float32)
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.empty((Hq, D), np.float32)
    if lib().orc_ref_faithful_decode_copy(_p(kc), _p(vc), T, Hkv, Hq, D, _p(kn), _p(vn), _p(q), scale, _p(out)):
        raise MemoryError("orc_ref_faithful_decode_copy")
    return out


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(n)


def set_setup_threads(n: int) -> None:
    """Threads that fill ref_faithful_batch's caches before its timed region
    (0: the current thread count)."""
    lib().orc_set_setup_threads(n)
