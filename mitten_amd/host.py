"""Python mirror of the engine's host-side KV bookkeeping (libmitten_kvhost.so).

Same names and argument meaning as the reference engine:

    KvCachePool    inference-engine/src/kv_pool.rs:4-69
    PageTable      inference-engine/src/kv_pool.rs:71-102
    RadixCache     inference-engine/src/radix_cache.rs:37-303

plus BlockManager, the page lifecycle that feeds the device pool (admission
with prefix match, decode-time growth, copy-on-write, promotion into the
tree, release, eviction and compaction), with per-block reference counts.

Error behaviour: where the reference returns None (allocation from an empty
pool, lookup of a missing entry) these return None; where it panics in
debug builds (freeing a page that is not in use, kv_pool.rs:41-44) they
raise DoubleFree.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._host_sigs import I32P, I64P, U32P, U64P

OK, INVALID_ARGUMENT, EXHAUSTED, NOT_IN_USE, BUFFER_TOO_SMALL, NOT_FOUND = range(6)


class HostError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class DoubleFree(HostError):
    """KvCachePool::free of a page that is not in use (kv_pool.rs:41-44)."""


class OutOfBlocks(HostError):
    """No free block (EngineError::OutOfKvPages)."""


def _lib_h():
    return _lib.host_lib()


def _check(status: int) -> None:
    if status == OK:
        return
    msg = (_lib_h().mkvh_last_error() or b"").decode(errors="replace")
    if status == NOT_IN_USE:
        raise DoubleFree(status, msg)
    if status == EXHAUSTED:
        raise OutOfBlocks(status, msg)
    raise HostError(status, msg)


def _u32(a, name: str = "ids") -> np.ndarray:
    """Token ids and page ids are u32: values outside [0, 2^32) are refused
    rather than wrapped by the cast."""
    x = np.asarray(a)
    if x.size:
        if x.dtype.kind not in "iu":
            raise HostError(INVALID_ARGUMENT, f"{name} must hold integers, not {x.dtype}")
        if (x.dtype.kind == "i" and int(x.min()) < 0) or int(x.max()) > 0xFFFFFFFF:
            raise HostError(INVALID_ARGUMENT, f"{name} holds a value outside u32")
    return np.ascontiguousarray(x, np.uint32)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


class _Handle:
    _destroy = ""

    def close(self) -> None:
        if getattr(self, "_h", None):
            getattr(_lib_h(), self._destroy)(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KvCachePool(_Handle):
    """LIFO page allocator (kv_pool.rs:4-69); pages come out 0, 1, 2, ..."""

    _destroy = "mkvh_kv_pool_destroy"

    def __init__(self, num_pages: int, page_size: int):
        h = ctypes.c_void_p()
        _check(_lib_h().mkvh_kv_pool_create(num_pages, page_size, ctypes.byref(h)))
        self._h = h
        self.num_pages = num_pages
        self.page_size = page_size

    def allocate(self, owner: int):
        """kv_pool.rs:30-37: a page id, or None when the pool is exhausted."""
        out = ctypes.c_uint32()
        st = _lib_h().mkvh_kv_pool_allocate(self._h, owner, ctypes.byref(out))
        if st == EXHAUSTED:
            return None
        _check(st)
        return out.value

    def free(self, page: int) -> None:
        """kv_pool.rs:40-47; raises DoubleFree where the reference debug-asserts."""
        _check(_lib_h().mkvh_kv_pool_free(self._h, page))

    def free_pages(self) -> int:
        return _lib_h().mkvh_kv_pool_free_pages(self._h)

    def total_pages(self) -> int:
        return _lib_h().mkvh_kv_pool_total_pages(self._h)

    def page_state(self, page: int):
        """(in_use, owner, refcount)."""
        iu, ow, rc = ctypes.c_int32(), ctypes.c_uint64(), ctypes.c_int32()
        _check(_lib_h().mkvh_kv_pool_page_state(self._h, page, ctypes.byref(iu), ctypes.byref(ow), ctypes.byref(rc)))
        return bool(iu.value), ow.value, rc.value

    def retain(self, page: int) -> None:
        _check(_lib_h().mkvh_kv_pool_retain(self._h, page))

    def release(self, page: int) -> bool:
        """Drops one reference; True when the page went back to the pool."""
        f = ctypes.c_int32()
        _check(_lib_h().mkvh_kv_pool_release(self._h, page, ctypes.byref(f)))
        return bool(f.value)

    @staticmethod
    def required_bytes(num_pages, page_size, num_layers, num_kv_heads, head_dim, dtype_bytes) -> int:
        """kv_pool.rs:58-68."""
        return _lib_h().mkvh_required_bytes(num_pages, page_size, num_layers, num_kv_heads, head_dim,
                                            dtype_bytes)


class PageTable(_Handle):
    """(request, slot) -> page (kv_pool.rs:71-102)."""

    _destroy = "mkvh_page_table_destroy"

    def __init__(self):
        h = ctypes.c_void_p()
        _check(_lib_h().mkvh_page_table_create(ctypes.byref(h)))
        self._h = h

    def insert(self, req_id: int, slot: int, page: int) -> None:
        _check(_lib_h().mkvh_page_table_insert(self._h, req_id, slot, page))

    def lookup(self, req_id: int, slot: int):
        out = ctypes.c_uint32()
        st = _lib_h().mkvh_page_table_lookup(self._h, req_id, slot, ctypes.byref(out))
        if st == NOT_FOUND:
            return None
        _check(st)
        return out.value

    def remove_request(self, req_id: int) -> list[int]:
        cap = 1 << 16
        while True:
            buf = np.empty(cap, np.uint32)
            n = ctypes.c_int64()
            st = _lib_h().mkvh_page_table_remove_request(self._h, req_id, _ptr(buf, U32P), cap, ctypes.byref(n))
            if st == BUFFER_TOO_SMALL:
                cap *= 4
                continue
            _check(st)
            return buf[: n.value].tolist()


class RadixCache(_Handle):
    """Radix prefix cache over u32 tokens (radix_cache.rs:37-303). Node ids are
    slab indices. Pages evicted by insert_prefix / promote_request (which the
    reference drops, radix_cache.rs:132-134) are kept for take_evicted()."""

    _destroy = "mkvh_radix_destroy"

    def __init__(self, page_size: int, max_pages: int):
        h = ctypes.c_void_p()
        _check(_lib_h().mkvh_radix_create(page_size, max_pages, ctypes.byref(h)))
        self._h = h
        self.page_size = page_size
        self._pending: list[int] = []

    def match_prefix(self, tokens):
        """(matched_len, pages, locked_node_ids); locks every matched node."""
        t = _u32(tokens, "tokens")
        cap = max(1, t.size // self.page_size)
        pages = np.empty(cap, np.uint32)
        nodes = np.empty(cap, np.uint64)
        ml, npg, nnd = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        _check(_lib_h().mkvh_radix_match_prefix(self._h, _ptr(t, U32P), t.size, ctypes.byref(ml), _ptr(pages, U32P),
                                                cap, ctypes.byref(npg), _ptr(nodes, U64P), cap, ctypes.byref(nnd)))
        return ml.value, pages[: npg.value].tolist(), nodes[: nnd.value].tolist()

    def insert_prefix(self, tokens, pages) -> None:
        t, p = _u32(tokens, "tokens"), _u32(pages, "pages")
        _check(_lib_h().mkvh_radix_insert_prefix(self._h, _ptr(t, U32P), t.size, _ptr(p, U32P), p.size))

    def unlock_nodes(self, node_ids) -> None:
        n = np.ascontiguousarray(node_ids, np.uint64)
        _check(_lib_h().mkvh_radix_unlock_nodes(self._h, _ptr(n, U64P), n.size))

    def _drain(self) -> list[int]:
        got = []
        while True:
            buf = np.empty(4096, np.uint32)
            n = ctypes.c_int64()
            _check(_lib_h().mkvh_radix_drain_evicted(self._h, _ptr(buf, U32P), buf.size, ctypes.byref(n)))
            got += buf[: n.value].tolist()
            if n.value < buf.size:
                return got

    def evict_pages(self, target_pages: int) -> list[int]:
        """radix_cache.rs:243-282: pages freed by LRU eviction of unlocked
        leaves (>= target unless no evictable leaf is left)."""
        n = ctypes.c_int64()
        _check(_lib_h().mkvh_radix_evict_pages(self._h, target_pages, ctypes.byref(n)))
        queued = self._pending + self._drain()
        cut = len(queued) - n.value
        self._pending = queued[:cut]
        return queued[cut:]

    def take_evicted(self) -> list[int]:
        """Pages evicted by insert_prefix / promote_request so far."""
        out = self._pending + self._drain()
        self._pending = []
        return out

    def promote_request(self, input_ids, device_len: int, kv_pages) -> None:
        """radix_cache.rs:287-294 (a Request's input_ids, device_len, kv_pages)."""
        t, p = _u32(input_ids, "input_ids"), _u32(kv_pages, "kv_pages")
        _check(_lib_h().mkvh_radix_promote_request(self._h, _ptr(t, U32P), t.size, device_len, _ptr(p, U32P),
                                                   p.size))

    def total_cached_pages(self) -> int:
        return _lib_h().mkvh_radix_total_cached_pages(self._h)

    def num_nodes(self) -> int:
        return _lib_h().mkvh_radix_num_nodes(self._h)


def schedule_prefill_chunks(budget: int, remaining) -> tuple[list[int], int]:
    """The chunking rule of PrefillAdder (inference-engine/src/prefill.rs:27-36,
    99-114) over in-progress prefills, in order: each gets min(remaining,
    budget - used) tokens until the budget is used up. Returns (chunks,
    tokens used)."""
    r = np.ascontiguousarray(remaining, np.int64)
    out, used = np.zeros(max(1, r.size), np.int64), ctypes.c_int64()
    _check(_lib_h().mkvh_schedule_prefill_chunks(budget, _ptr(r, I64P), r.size, _ptr(out, I64P),
                                                 ctypes.byref(used)))
    return [int(c) for c in out[:r.size]], used.value


class BlockManager(_Handle):
    """Block tables of live sequences over a pool of `num_blocks` device blocks,
    with the radix tree caching up to `max_cached_pages` full pages."""

    _destroy = "mkvh_bm_destroy"

    def __init__(self, num_blocks: int, page_size: int = 16, max_cached_pages: int | None = None):
        h = ctypes.c_void_p()
        mc = num_blocks if max_cached_pages is None else max_cached_pages
        _check(_lib_h().mkvh_bm_create(num_blocks, page_size, mc, ctypes.byref(h)))
        self._h = h
        self.num_blocks = num_blocks
        self.page_size = page_size

    def admit(self, seq: int, tokens) -> int:
        """Admission (prefill.rs:39-81); returns the cached prefix length."""
        t = _u32(tokens, "tokens")
        out = ctypes.c_int64()
        _check(_lib_h().mkvh_bm_admit(self._h, seq, _ptr(t, U32P), t.size, ctypes.byref(out)))
        return out.value

    def fork(self, parent: int, child: int) -> None:
        _check(_lib_h().mkvh_bm_fork(self._h, parent, child))

    def append(self, seq: int, n_new: int):
        """(slots int32[n_new], cow pairs list[(src, dst)])."""
        slots = np.empty(max(1, n_new), np.int32)
        src, dst, n = np.empty(1, np.int32), np.empty(1, np.int32), ctypes.c_int32()
        _check(_lib_h().mkvh_bm_append(self._h, seq, n_new, _ptr(slots, I32P), _ptr(src, I32P), _ptr(dst, I32P),
                                       ctypes.byref(n)))
        return slots[:n_new], [(int(src[0]), int(dst[0]))] if n.value else []

    def schedule_prefill(self, budget: int, in_progress, waiting):
        """PrefillAdder::run (prefill.rs:21-114) on these books: in-progress
        prefills (sequence ids, in order) first, then waiting requests
        [(seq, prompt tokens), ...] admitted in order while budget remains,
        each chunk min(remaining, budget - used). Returns (chunks of the
        in-progress sequences, chunks of the waiting ones, number admitted
        (a prefix of `waiting`), their cached lengths)."""
        ip = np.ascontiguousarray(list(in_progress), np.uint64)
        wseq = np.ascontiguousarray([s for s, _ in waiting], np.uint64)
        toks = [_u32(t, "prompt tokens") for _, t in waiting]
        windptr = np.zeros(len(toks) + 1, np.int64)
        np.cumsum([t.size for t in toks], out=windptr[1:])
        wtok = np.concatenate(toks) if toks else np.zeros(1, np.uint32)
        chunks = np.zeros(max(1, ip.size + wseq.size), np.int64)
        cached = np.zeros(max(1, wseq.size), np.int64)
        n_adm = ctypes.c_int32()
        _check(_lib_h().mkvh_bm_schedule_prefill(
            self._h, budget, _ptr(ip, U64P), ip.size, _ptr(wseq, U64P), _ptr(windptr, I64P), _ptr(wtok, U32P),
            wseq.size, _ptr(chunks, I64P), ctypes.byref(n_adm), _ptr(cached, I64P)))
        k = n_adm.value
        return ([int(c) for c in chunks[:ip.size]], [int(c) for c in chunks[ip.size:ip.size + wseq.size]], k,
                [int(c) for c in cached[:k]])

    def promote(self, seq: int, tokens) -> None:
        t = _u32(tokens, "tokens")
        _check(_lib_h().mkvh_bm_promote(self._h, seq, _ptr(t, U32P), t.size))

    def release(self, seq: int) -> None:
        _check(_lib_h().mkvh_bm_release(self._h, seq))

    def evict(self, target_pages: int) -> int:
        n = ctypes.c_int64()
        _check(_lib_h().mkvh_bm_evict(self._h, target_pages, ctypes.byref(n)))
        return n.value

    def plan_compaction(self):
        """(src int32[n], dst int32[n]) block moves; tables are rewritten."""
        cap = self.num_blocks
        src, dst, n = np.empty(max(1, cap), np.int32), np.empty(max(1, cap), np.int32), ctypes.c_int64()
        _check(_lib_h().mkvh_bm_plan_compaction(self._h, _ptr(src, I32P), _ptr(dst, I32P), cap, ctypes.byref(n)))
        return src[: n.value].copy(), dst[: n.value].copy()

    def seq_len(self, seq: int) -> int:
        out = ctypes.c_int64()
        _check(_lib_h().mkvh_bm_seq_len(self._h, seq, ctypes.byref(out)))
        return out.value

    def table(self, seq: int) -> np.ndarray:
        cap = self.num_blocks
        buf, n = np.empty(max(1, cap), np.int32), ctypes.c_int64()
        _check(_lib_h().mkvh_bm_table(self._h, seq, _ptr(buf, I32P), cap, ctypes.byref(n)))
        return buf[: n.value].copy()

    def batch(self, seqs):
        """(block_indptr int32[B+1], block_ids int32[nnz], ctx_lens int32[B])."""
        s = np.ascontiguousarray(seqs, np.uint64)
        indptr = np.empty(s.size + 1, np.int32)
        ctx = np.empty(max(1, s.size), np.int32)
        cap = self.num_blocks * max(1, s.size)
        cap = min(cap, 1 << 26)
        ids = np.empty(max(1, cap), np.int32)
        _check(_lib_h().mkvh_bm_batch(self._h, _ptr(s, U64P), s.size, _ptr(indptr, I32P), _ptr(ids, I32P), cap,
                                      _ptr(ctx, I32P)))
        return indptr, ids[: indptr[-1]].copy(), ctx[: s.size].copy()

    def batch_shared_prefix(self, seqs):
        """The step's tables split at the blocks every sequence shares: see
        split_shared_prefix."""
        return split_shared_prefix(*self.batch(seqs))

    def free_blocks(self) -> int:
        return _lib_h().mkvh_bm_free_blocks(self._h)

    def live_blocks(self) -> int:
        return _lib_h().mkvh_bm_live_blocks(self._h)

    def refcount(self, block: int) -> int:
        return _lib_h().mkvh_bm_refcount(self._h, block)

    def cached_pages(self) -> int:
        return _lib_h().mkvh_bm_cached_pages(self._h)

    def check_invariants(self) -> None:
        _check(_lib_h().mkvh_bm_check_invariants(self._h))


def split_shared_prefix(block_indptr, block_ids, ctx_lens):
    """Splits a step's block tables at the longest run of leading block ids
    that every table holds (radix sharing hands the same pages to each
    request that matched a prefix, inference-engine/src/radix_cache.rs:64-117),
    limited to pages that are full before each sequence's last token.
    Returns (prefix_ids int32[n], suffix_indptr int32[B+1], suffix_ids int32,
    suffix_lens int32[B]) for DeviceKvPool.plan_suffixes and
    decode_step_shared_prefix; n = 0 when nothing is shared."""
    ip = np.asarray(block_indptr, np.int64)
    ids = np.asarray(block_ids, np.int32)
    ctx = np.asarray(ctx_lens, np.int64)
    B = ctx.size
    lens = ip[1:] - ip[:-1]
    limit = int(min(((ctx - 1) // 16).min(), lens.min())) if B else 0
    n = 0
    if limit > 0:
        lead = ids[ip[:-1, None] + np.arange(limit)[None, :]]  # [B, limit] leading ids
        same = (lead == lead[0]).all(axis=0)
        n = limit if same.all() else int(np.argmin(same))
    suffix_indptr = (ip - n * np.arange(B + 1)).astype(np.int32)
    keep = np.ones(ids.size, bool)
    for b in range(B):
        keep[ip[b]:ip[b] + n] = False
    return (ids[ip[0]:ip[0] + n].copy() if B else ids[:0].copy(), suffix_indptr, ids[keep],
            (ctx - 16 * n).astype(np.int32))
