"""ctypes signatures of libmitten_kvhost.so (include/mitten_kv_host.h)."""
import ctypes

P = ctypes.c_void_p
i32, i64, u32, u64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64
c_int = ctypes.c_int
PP = ctypes.POINTER(P)
I32P, I64P, U32P, U64P = (ctypes.POINTER(t) for t in (i32, i64, u32, u64))

HOST_SIGNATURES = {
    "mkvh_last_error": (ctypes.c_char_p, []),
    "mkvh_required_bytes": (u64, [u64, u64, u64, u64, u64, u64]),
    "mkvh_kv_pool_create": (c_int, [i64, i32, PP]),
    "mkvh_kv_pool_destroy": (None, [P]),
    "mkvh_kv_pool_allocate": (c_int, [P, u64, U32P]),
    "mkvh_kv_pool_free": (c_int, [P, u32]),
    "mkvh_kv_pool_free_pages": (i64, [P]),
    "mkvh_kv_pool_total_pages": (i64, [P]),
    "mkvh_kv_pool_page_state": (c_int, [P, u32, I32P, U64P, I32P]),
    "mkvh_kv_pool_retain": (c_int, [P, u32]),
    "mkvh_kv_pool_release": (c_int, [P, u32, I32P]),
    "mkvh_page_table_create": (c_int, [PP]),
    "mkvh_page_table_destroy": (None, [P]),
    "mkvh_page_table_insert": (c_int, [P, u64, i64, u32]),
    "mkvh_page_table_lookup": (c_int, [P, u64, i64, U32P]),
    "mkvh_page_table_remove_request": (c_int, [P, u64, U32P, i64, I64P]),
    "mkvh_radix_create": (c_int, [i32, i64, PP]),
    "mkvh_radix_destroy": (None, [P]),
    "mkvh_radix_match_prefix": (c_int, [P, U32P, i64, I64P, U32P, i64, I64P, U64P, i64, I64P]),
    "mkvh_radix_insert_prefix": (c_int, [P, U32P, i64, U32P, i64]),
    "mkvh_radix_unlock_nodes": (c_int, [P, U64P, i64]),
    "mkvh_radix_evict_pages": (c_int, [P, i64, I64P]),
    "mkvh_radix_drain_evicted": (c_int, [P, U32P, i64, I64P]),
    "mkvh_radix_promote_request": (c_int, [P, U32P, i64, i64, U32P, i64]),
    "mkvh_radix_total_cached_pages": (i64, [P]),
    "mkvh_radix_num_nodes": (i64, [P]),
    "mkvh_bm_create": (c_int, [i64, i32, i64, PP]),
    "mkvh_bm_destroy": (None, [P]),
    "mkvh_bm_admit": (c_int, [P, u64, U32P, i64, I64P]),
    "mkvh_bm_fork": (c_int, [P, u64, u64]),
    "mkvh_bm_append": (c_int, [P, u64, i32, I32P, I32P, I32P, I32P]),
    "mkvh_schedule_prefill_chunks": (c_int, [i64, I64P, i32, I64P, I64P]),
    "mkvh_bm_schedule_prefill": (c_int, [P, i64, U64P, i32, U64P, I64P, U32P, i32, I64P, ctypes.POINTER(i32), I64P]),
    "mkvh_bm_promote": (c_int, [P, u64, U32P, i64]),
    "mkvh_bm_release": (c_int, [P, u64]),
    "mkvh_bm_evict": (c_int, [P, i64, I64P]),
    "mkvh_bm_plan_compaction": (c_int, [P, I32P, I32P, i64, I64P]),
    "mkvh_bm_seq_len": (c_int, [P, u64, I64P]),
    "mkvh_bm_table": (c_int, [P, u64, I32P, i64, I64P]),
    "mkvh_bm_batch": (c_int, [P, U64P, i32, I32P, I32P, i64, I32P]),
    "mkvh_bm_free_blocks": (i64, [P]),
    "mkvh_bm_live_blocks": (i64, [P]),
    "mkvh_bm_refcount": (i32, [P, u32]),
    "mkvh_bm_cached_pages": (i64, [P]),
    "mkvh_bm_check_invariants": (c_int, [P]),
}
