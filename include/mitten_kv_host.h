/*
 * mitten_kv_host.h — C ABI of the host-side paged-KV bookkeeping
 * (libmitten_kvhost.so, plain C++, no device code).
 *
 * Restates the engine's page allocator, page table and radix prefix cache
 * (inference-engine/src/kv_pool.rs, radix_cache.rs) with their reference
 * semantics, and adds the block manager that drives the device pool: per-block
 * reference counts, decode-time block growth, copy-on-write of shared blocks
 * and pool compaction plans. The block manager emits exactly the metadata the
 * device operations of mitten_kv.h consume: slot mappings, CSR block tables
 * and (src, dst) block-copy pairs.
 *
 * Every function returns an mkvh_status; messages via mkvh_last_error().
 * Objects are not thread-safe (the engine owns them on its scheduler thread).
 */
#ifndef MITTEN_KV_HOST_H
#define MITTEN_KV_HOST_H

#include <stdint.h>

#ifndef MKVH_API
#define MKVH_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MKVH_OK = 0,
  MKVH_ERR_INVALID_ARGUMENT = 1,
  MKVH_ERR_EXHAUSTED = 2,        /* no free page (KvCachePool::allocate -> None) */
  MKVH_ERR_NOT_IN_USE = 3,       /* free of a page that is not in use (kv_pool.rs:41-44) */
  MKVH_ERR_BUFFER_TOO_SMALL = 4, /* output capacity too small; nothing was changed */
  MKVH_ERR_NOT_FOUND = 5         /* unknown sequence / page-table entry */
} mkvh_status;

MKVH_API const char *mkvh_last_error(void);

/* KvCachePool::required_bytes (kv_pool.rs:58-68). */
MKVH_API uint64_t mkvh_required_bytes(uint64_t num_pages, uint64_t page_size, uint64_t num_layers,
                                      uint64_t num_kv_heads, uint64_t head_dim,
                                      uint64_t dtype_bytes);

/* ---- KvCachePool (inference-engine/src/kv_pool.rs:4-69) ------------------ */
typedef struct mkvh_kv_pool mkvh_kv_pool;

/* KvCachePool::new (kv_pool.rs:18-27): LIFO free stack, pages come out 0,1,2,... */
MKVH_API int mkvh_kv_pool_create(int64_t num_pages, int32_t page_size, mkvh_kv_pool **out);
MKVH_API void mkvh_kv_pool_destroy(mkvh_kv_pool *pool);
/* allocate (kv_pool.rs:30-37): MKVH_ERR_EXHAUSTED where the reference returns None.
 * A fresh page has reference count 1. */
MKVH_API int mkvh_kv_pool_allocate(mkvh_kv_pool *pool, uint64_t owner, uint32_t *out_page);
/* free (kv_pool.rs:40-47): MKVH_ERR_NOT_IN_USE where the reference's
 * debug_assert fires (double free); ignores the reference count. */
MKVH_API int mkvh_kv_pool_free(mkvh_kv_pool *pool, uint32_t page);
MKVH_API int64_t mkvh_kv_pool_free_pages(const mkvh_kv_pool *pool);
MKVH_API int64_t mkvh_kv_pool_total_pages(const mkvh_kv_pool *pool);
MKVH_API int mkvh_kv_pool_page_state(const mkvh_kv_pool *pool, uint32_t page, int32_t *in_use,
                                     uint64_t *owner, int32_t *refcount);
/* Reference counting (the fix for radix-held pages being freed twice):
 * retain adds a holder; release drops one and frees the page at zero. */
MKVH_API int mkvh_kv_pool_retain(mkvh_kv_pool *pool, uint32_t page);
MKVH_API int mkvh_kv_pool_release(mkvh_kv_pool *pool, uint32_t page, int32_t *out_freed);

/* ---- PageTable (kv_pool.rs:71-102) ---------------------------------------- */
typedef struct mkvh_page_table mkvh_page_table;

MKVH_API int mkvh_page_table_create(mkvh_page_table **out);
MKVH_API void mkvh_page_table_destroy(mkvh_page_table *pt);
MKVH_API int mkvh_page_table_insert(mkvh_page_table *pt, uint64_t req, int64_t slot, uint32_t page);
/* MKVH_ERR_NOT_FOUND where the reference returns None. */
MKVH_API int mkvh_page_table_lookup(const mkvh_page_table *pt, uint64_t req, int64_t slot,
                                    uint32_t *out_page);
/* Removes every entry of `req`; pages in ascending slot order. */
MKVH_API int mkvh_page_table_remove_request(mkvh_page_table *pt, uint64_t req, uint32_t *out_pages,
                                            int64_t cap, int64_t *out_n);

/* ---- RadixCache (inference-engine/src/radix_cache.rs:37-303) --------------- */
typedef struct mkvh_radix mkvh_radix;

MKVH_API int mkvh_radix_create(int32_t page_size, int64_t max_pages, mkvh_radix **out);
MKVH_API void mkvh_radix_destroy(mkvh_radix *r);
/* match_prefix (radix_cache.rs:64-117): page-aligned longest prefix; locks
 * every matched node. Capacities must be >= n_tokens / page_size. */
MKVH_API int mkvh_radix_match_prefix(mkvh_radix *r, const uint32_t *tokens, int64_t n_tokens,
                                     int64_t *out_matched_len, uint32_t *out_pages,
                                     int64_t pages_cap, int64_t *out_n_pages, uint64_t *out_nodes,
                                     int64_t nodes_cap, int64_t *out_n_nodes);
/* insert_prefix (radix_cache.rs:123-187): full pages only. Pages evicted to
 * make room are queued (the reference drops them, radix_cache.rs:132-134);
 * take them with mkvh_radix_drain_evicted. */
MKVH_API int mkvh_radix_insert_prefix(mkvh_radix *r, const uint32_t *tokens, int64_t n_tokens,
                                      const uint32_t *pages, int64_t n_pages);
MKVH_API int mkvh_radix_unlock_nodes(mkvh_radix *r, const uint64_t *nodes, int64_t n);
/* evict_pages (radix_cache.rs:243-282): LRU unlocked leaves until >= target
 * pages are freed (or nothing is evictable); the pages are queued. */
MKVH_API int mkvh_radix_evict_pages(mkvh_radix *r, int64_t target, int64_t *out_n_freed);
MKVH_API int mkvh_radix_drain_evicted(mkvh_radix *r, uint32_t *out_pages, int64_t cap,
                                      int64_t *out_n);
/* promote_request (radix_cache.rs:287-294). */
MKVH_API int mkvh_radix_promote_request(mkvh_radix *r, const uint32_t *input_ids, int64_t n_input,
                                        int64_t device_len, const uint32_t *kv_pages,
                                        int64_t n_pages);
MKVH_API int64_t mkvh_radix_total_cached_pages(const mkvh_radix *r);
MKVH_API int64_t mkvh_radix_num_nodes(const mkvh_radix *r);

/* ---- Block manager: the engine's page lifecycle with the build's fixes ------ */
typedef struct mkvh_block_manager mkvh_block_manager;

/* num_blocks device blocks of page_size tokens; the radix tree may cache up
 * to max_cached_pages of them. */
MKVH_API int mkvh_bm_create(int64_t num_blocks, int32_t page_size, int64_t max_cached_pages,
                            mkvh_block_manager **out);
MKVH_API void mkvh_bm_destroy(mkvh_block_manager *bm);
/* Admission (prefill.rs:39-81): radix match of the prompt (full pages), lock
 * the matched nodes, share the matched blocks, allocate the remaining
 * ceil(n/page_size) blocks, evicting LRU tree leaves on a deficit.
 * MKVH_ERR_EXHAUSTED (and no change) when the pool cannot hold the prompt.
 * *out_cached_len = prompt tokens whose K/V are already in the pool. The
 * sequence's length becomes *out_cached_len; append the rest. */
MKVH_API int mkvh_bm_admit(mkvh_block_manager *bm, uint64_t seq, const uint32_t *tokens,
                           int64_t n_tokens, int64_t *out_cached_len);
/* New sequence sharing every block of `parent` (refcount + 1 each), including
 * a partly filled last block: parallel sampling / forked decoding. */
MKVH_API int mkvh_bm_fork(mkvh_block_manager *bm, uint64_t parent, uint64_t child);
/* Slots for n_new tokens at positions [len, len + n_new): a block is
 * allocated whenever a position starts one (decode-time growth). Every block
 * in the written range that is shared (refcount > 1: a fork, including one
 * made before the prompt was written) is replaced by a private block first.
 * Only the block holding position len, when it already holds rows of this
 * sequence (len % page_size != 0), needs its contents: that pair is
 * returned in (cow_src, cow_dst) (0 or 1 pairs; required outputs when it
 * occurs) and must run (mkv_copy_blocks) before the append. The last holder
 * of a shared block writes in place. */
MKVH_API int mkvh_bm_append(mkvh_block_manager *bm, uint64_t seq, int32_t n_new, int32_t *out_slots,
                            int32_t *out_cow_src, int32_t *out_cow_dst, int32_t *out_n_cow);
/* The chunking rule of PrefillAdder (inference-engine/src/prefill.rs:27-36,
 * 99-114) over requests whose prefill is in progress, in order, with no
 * pool involved: request i, with remaining[i] prompt tokens still to write,
 * gets out_chunks[i] = min(remaining[i], budget - used) tokens; once the
 * budget is used up the loop stops and the rest get 0, as does a request
 * with nothing remaining. *out_used = tokens scheduled. budget is the
 * engine's max_prefill_tokens_per_iter minus the step's decode tokens
 * (scheduler.rs:14-18). */
MKVH_API int mkvh_schedule_prefill_chunks(int64_t budget, const int64_t *remaining, int32_t n,
                                          int64_t *out_chunks, int64_t *out_used);
/* PrefillAdder::run (prefill.rs:21-114) on the block manager's books.
 * 1. in_progress[0..n_in_progress): admitted sequences whose prompt is not
 *    all written, in order; remaining = prompt length - tokens written; the
 *    chunk rule above.
 * 2. Then, while budget remains, waiting requests in order: request i's
 *    prompt is waiting_tokens[waiting_indptr[i] .. waiting_indptr[i+1]); it
 *    is admitted under sequence id waiting[i] as mkvh_bm_admit does (evict
 *    the deficit once, radix match, allocate the rest), and gets its chunk by
 *    the same rule from its cached length on. The first request the pool
 *    cannot hold ends admission (the reference's `break`), as does the
 *    budget.
 * out_chunks[n_in_progress + n_waiting]: each request's chunk this step
 * (0: none; an admitted request whose whole prompt was cached gets 0, as in
 * the reference). *out_n_admitted: waiting requests admitted (a prefix of
 * the list: the engine moves them to its prefilling list);
 * out_cached_lens[i] (i < *out_n_admitted): their radix hits. Append each
 * chunk with mkvh_bm_append. */
MKVH_API int mkvh_bm_schedule_prefill(mkvh_block_manager *bm, int64_t budget, const uint64_t *in_progress,
                                      int32_t n_in_progress, const uint64_t *waiting,
                                      const int64_t *waiting_indptr, const uint32_t *waiting_tokens,
                                      int32_t n_waiting, int64_t *out_chunks, int32_t *out_n_admitted,
                                      int64_t *out_cached_lens);
/* Prefill complete (scheduler.rs:117): full pages enter the tree; the tree
 * holds its own reference to each page it adopts. */
MKVH_API int mkvh_bm_promote(mkvh_block_manager *bm, uint64_t seq, const uint32_t *tokens,
                             int64_t n_tokens);
/* Done / Aborted (scheduler.rs:164-172, decode.rs:20-33): unlock matched
 * nodes and drop the sequence's references; pages the tree holds survive. */
MKVH_API int mkvh_bm_release(mkvh_block_manager *bm, uint64_t seq);
/* LRU eviction of tree leaves; blocks whose last reference goes are freed. */
MKVH_API int mkvh_bm_evict(mkvh_block_manager *bm, int64_t target_pages, int64_t *out_freed_blocks);
/* Compaction plan: every live block with id >= live_count moves to a free id
 * below live_count; block tables and tree pages are rewritten. Returns the
 * moves for mkv_copy_blocks (sources and destinations are disjoint).
 * out_src / out_dst (capacity cap) are required whenever a move is needed:
 * otherwise nothing changes and MKVH_ERR_INVALID_ARGUMENT is returned. */
MKVH_API int mkvh_bm_plan_compaction(mkvh_block_manager *bm, int32_t *out_src, int32_t *out_dst,
                                     int64_t cap, int64_t *out_n);
MKVH_API int mkvh_bm_seq_len(const mkvh_block_manager *bm, uint64_t seq, int64_t *out_len);
MKVH_API int mkvh_bm_table(const mkvh_block_manager *bm, uint64_t seq, int32_t *out_blocks,
                           int64_t cap, int64_t *out_n);
/* CSR block tables + context lengths (tokens written) of a batch, in order. */
MKVH_API int mkvh_bm_batch(const mkvh_block_manager *bm, const uint64_t *seqs, int32_t n_seqs,
                           int32_t *out_indptr, int32_t *out_ids, int64_t ids_cap,
                           int32_t *out_ctx_lens);
MKVH_API int64_t mkvh_bm_free_blocks(const mkvh_block_manager *bm);
MKVH_API int64_t mkvh_bm_live_blocks(const mkvh_block_manager *bm);
MKVH_API int32_t mkvh_bm_refcount(const mkvh_block_manager *bm, uint32_t block);
MKVH_API int64_t mkvh_bm_cached_pages(const mkvh_block_manager *bm);
/* Consistency audit: every live block's refcount equals its holders (sequence
 * tables + tree), free + live = total, no free block is referenced. */
MKVH_API int mkvh_bm_check_invariants(const mkvh_block_manager *bm);

#ifdef __cplusplus
}
#endif

#endif /* MITTEN_KV_HOST_H */
