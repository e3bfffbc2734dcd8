//! Raw FFI of `libmitten_kvhost.so` (`include/mitten_kv_host.h`): the host
//! bookkeeping of the paged KV path (page allocator, page table, radix
//! prefix cache, and the block manager with per-block reference counts,
//! decode-time growth, copy-on-write, compaction and the prefill budget
//! rule). Plain C++, no device code. Not thread-safe: one owner thread.
#![allow(non_camel_case_types)]
use std::ffi::c_char;

pub const MKVH_OK: i32 = 0;
pub const MKVH_ERR_INVALID_ARGUMENT: i32 = 1;
pub const MKVH_ERR_EXHAUSTED: i32 = 2;
pub const MKVH_ERR_NOT_IN_USE: i32 = 3;
pub const MKVH_ERR_BUFFER_TOO_SMALL: i32 = 4;
pub const MKVH_ERR_NOT_FOUND: i32 = 5;
#[repr(C)] pub struct mkvh_kv_pool { _p: [u8; 0] }
#[repr(C)] pub struct mkvh_page_table { _p: [u8; 0] }
#[repr(C)] pub struct mkvh_radix { _p: [u8; 0] }
#[repr(C)] pub struct mkvh_block_manager { _p: [u8; 0] }

extern "C" {
    pub fn mkvh_last_error() -> *const c_char;
    pub fn mkvh_required_bytes(num_pages: u64, page_size: u64, num_layers: u64, num_kv_heads: u64,
                               head_dim: u64, dtype_bytes: u64) -> u64;
    pub fn mkvh_kv_pool_create(num_pages: i64, page_size: i32, out: *mut *mut mkvh_kv_pool) -> i32;
    pub fn mkvh_kv_pool_destroy(pool: *mut mkvh_kv_pool);
    pub fn mkvh_kv_pool_allocate(pool: *mut mkvh_kv_pool, owner: u64, out_page: *mut u32) -> i32;
    pub fn mkvh_kv_pool_free(pool: *mut mkvh_kv_pool, page: u32) -> i32;
    pub fn mkvh_kv_pool_free_pages(pool: *const mkvh_kv_pool) -> i64;
    pub fn mkvh_kv_pool_total_pages(pool: *const mkvh_kv_pool) -> i64;
    pub fn mkvh_kv_pool_page_state(pool: *const mkvh_kv_pool, page: u32, in_use: *mut i32, owner: *mut u64,
                                   refcount: *mut i32) -> i32;
    pub fn mkvh_kv_pool_retain(pool: *mut mkvh_kv_pool, page: u32) -> i32;
    pub fn mkvh_kv_pool_release(pool: *mut mkvh_kv_pool, page: u32, out_freed: *mut i32) -> i32;
    pub fn mkvh_page_table_create(out: *mut *mut mkvh_page_table) -> i32;
    pub fn mkvh_page_table_destroy(pt: *mut mkvh_page_table);
    pub fn mkvh_page_table_insert(pt: *mut mkvh_page_table, req: u64, slot: i64, page: u32) -> i32;
    pub fn mkvh_page_table_lookup(pt: *const mkvh_page_table, req: u64, slot: i64, out_page: *mut u32) -> i32;
    pub fn mkvh_page_table_remove_request(pt: *mut mkvh_page_table, req: u64, out_pages: *mut u32, cap: i64,
                                          out_n: *mut i64) -> i32;
    pub fn mkvh_radix_create(page_size: i32, max_pages: i64, out: *mut *mut mkvh_radix) -> i32;
    pub fn mkvh_radix_destroy(r: *mut mkvh_radix);
    pub fn mkvh_radix_match_prefix(r: *mut mkvh_radix, tokens: *const u32, n_tokens: i64,
                                   out_matched_len: *mut i64, out_pages: *mut u32, pages_cap: i64,
                                   out_n_pages: *mut i64, out_nodes: *mut u64, nodes_cap: i64,
                                   out_n_nodes: *mut i64) -> i32;
    pub fn mkvh_radix_insert_prefix(r: *mut mkvh_radix, tokens: *const u32, n_tokens: i64, pages: *const u32,
                                    n_pages: i64) -> i32;
    pub fn mkvh_radix_unlock_nodes(r: *mut mkvh_radix, nodes: *const u64, n: i64) -> i32;
    pub fn mkvh_radix_evict_pages(r: *mut mkvh_radix, target: i64, out_n_freed: *mut i64) -> i32;
    pub fn mkvh_radix_drain_evicted(r: *mut mkvh_radix, out_pages: *mut u32, cap: i64,
                                    out_n: *mut i64) -> i32;
    pub fn mkvh_radix_promote_request(r: *mut mkvh_radix, input_ids: *const u32, n_input: i64,
                                      device_len: i64, kv_pages: *const u32, n_pages: i64) -> i32;
    pub fn mkvh_radix_total_cached_pages(r: *const mkvh_radix) -> i64;
    pub fn mkvh_radix_num_nodes(r: *const mkvh_radix) -> i64;
    pub fn mkvh_bm_create(num_blocks: i64, page_size: i32, max_cached_pages: i64,
                          out: *mut *mut mkvh_block_manager) -> i32;
    pub fn mkvh_bm_destroy(bm: *mut mkvh_block_manager);
    pub fn mkvh_bm_admit(bm: *mut mkvh_block_manager, seq: u64, tokens: *const u32, n_tokens: i64,
                         out_cached_len: *mut i64) -> i32;
    pub fn mkvh_bm_fork(bm: *mut mkvh_block_manager, parent: u64, child: u64) -> i32;
    pub fn mkvh_bm_append(bm: *mut mkvh_block_manager, seq: u64, n_new: i32, out_slots: *mut i32,
                          out_cow_src: *mut i32, out_cow_dst: *mut i32, out_n_cow: *mut i32) -> i32;
    pub fn mkvh_schedule_prefill_chunks(budget: i64, remaining: *const i64, n: i32, out_chunks: *mut i64,
                                        out_used: *mut i64) -> i32;
    pub fn mkvh_bm_schedule_prefill(bm: *mut mkvh_block_manager, budget: i64, in_progress: *const u64,
                                    n_in_progress: i32, waiting: *const u64, waiting_indptr: *const i64,
                                    waiting_tokens: *const u32, n_waiting: i32, out_chunks: *mut i64,
                                    out_n_admitted: *mut i32, out_cached_lens: *mut i64) -> i32;
    pub fn mkvh_bm_promote(bm: *mut mkvh_block_manager, seq: u64, tokens: *const u32, n_tokens: i64) -> i32;
    pub fn mkvh_bm_release(bm: *mut mkvh_block_manager, seq: u64) -> i32;
    pub fn mkvh_bm_evict(bm: *mut mkvh_block_manager, target_pages: i64, out_freed_blocks: *mut i64) -> i32;
    pub fn mkvh_bm_plan_compaction(bm: *mut mkvh_block_manager, out_src: *mut i32, out_dst: *mut i32,
                                   cap: i64, out_n: *mut i64) -> i32;
    pub fn mkvh_bm_seq_len(bm: *const mkvh_block_manager, seq: u64, out_len: *mut i64) -> i32;
    pub fn mkvh_bm_table(bm: *const mkvh_block_manager, seq: u64, out_blocks: *mut i32, cap: i64,
                         out_n: *mut i64) -> i32;
    pub fn mkvh_bm_batch(bm: *const mkvh_block_manager, seqs: *const u64, n_seqs: i32, out_indptr: *mut i32,
                         out_ids: *mut i32, ids_cap: i64, out_ctx_lens: *mut i32) -> i32;
    pub fn mkvh_bm_free_blocks(bm: *const mkvh_block_manager) -> i64;
    pub fn mkvh_bm_live_blocks(bm: *const mkvh_block_manager) -> i64;
    pub fn mkvh_bm_refcount(bm: *const mkvh_block_manager, block: u32) -> i32;
    pub fn mkvh_bm_cached_pages(bm: *const mkvh_block_manager) -> i64;
    pub fn mkvh_bm_check_invariants(bm: *const mkvh_block_manager) -> i32;
}
