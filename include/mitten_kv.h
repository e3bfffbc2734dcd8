/*
 * mitten_kv.h — C ABI of the MI355X paged-KV library (libmitten_kv.so).
 *
 * The library owns the device KV pool (the inference backend's device-buffer
 * type) and runs the four data-plane operations of the engine's paged-KV path
 * as hand-written gfx950 HIP kernels:
 *
 *   append            scatter new K/V rows into block slots (slot mapping)
 *   gather            block table -> contiguous per-sequence K/V
 *   copy_blocks       copy-on-write block copies and batched block moves
 *   decode_attention  GQA/MQA paged decode attention straight from the pool
 *   extend_attention  causal attention of a chunk of new tokens (chunked prefill)
 *   qk_norm_rope_append  q/k RMSNorm + partial RoPE, fused with the K/V append
 *   wire_export / wire_import  blocks to / from a checksummed byte payload
 *                     (offload to host or disk, handoff between pools)
 *
 * Pool layout in HBM (design/rust-inference-engine-design.md:1380-1387):
 *   [num_layers][2 (K then V)][num_blocks][page_size][num_kv_heads][head_dim]
 * A slot id is block * page_size + offset_in_block.
 *
 * Conventions
 *   - Every function returns an mkv_status (0 = MKV_OK). On failure a message
 *     is available from mkv_last_error() (thread-local). No C++ exception and
 *     no abort crosses this boundary.
 *   - Pointers named d_* are device pointers (HBM), 16-byte aligned; h_* are
 *     host pointers. Metadata comes in two forms:
 *       * host arrays in the engine's own form (the *_host entry points and
 *         mkv_decode_plan_build_tables): page ids are u32 (PageIndex,
 *         inference-engine/src/request.rs:6), a batch's page tables
 *         (Vec<Vec<u32>>, inference-backend/src/batch.rs:24-26) are passed
 *         as a CSR pair u32 indptr[B+1] / ids[indptr[B]]. They are validated
 *         on the host (a bad id returns MKV_ERR_INVALID_ARGUMENT and nothing
 *         is launched) and copied before the call returns: the caller keeps
 *         ownership and may reuse the arrays at once. The library uploads
 *         them on `stream` ahead of the launch;
 *       * device int32 arrays (the other entry points), read by the kernels
 *         when they run. The mkv_validate_* functions check such arrays on
 *         the host.
 *   - Kernels bound-check every slot and block id they dereference against
 *     the pool; an out-of-range id is skipped (never dereferenced) and
 *     recorded in the pool's device error word, read by mkv_pool_check().
 *   - `stream` is a hipStream_t (NULL = the null stream). Operations are
 *     asynchronous on that stream. A pool is not thread-safe: one caller
 *     thread at a time (the engine drives it from its single GPU thread,
 *     inference-api/src/main.rs:84-91).
 */
#ifndef MITTEN_KV_H
#define MITTEN_KV_H

#include <stddef.h>
#include <stdint.h>

#ifndef MKV_API
#define MKV_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Mapping onto the engine's error type
 * (inference-backend/src/error.rs:3-13):
 *   MKV_ERR_OUT_OF_MEMORY -> EngineError::OutOfKvPages
 *   everything else       -> EngineError::Backend(mkv_last_error()) */
typedef enum {
  MKV_OK = 0,
  MKV_ERR_INVALID_ARGUMENT = 1,
  MKV_ERR_OUT_OF_MEMORY = 2,
  MKV_ERR_HIP = 3,
  MKV_ERR_DEVICE_INDEX = 4, /* a kernel met an out-of-range id (mkv_pool_check) */
  MKV_ERR_NO_DEVICE = 5
} mkv_status;

typedef enum { MKV_DTYPE_F32 = 0, MKV_DTYPE_BF16 = 1 } mkv_dtype;

/* Bits of the device error word (mkv_pool_check). */
enum {
  MKV_DEVERR_SLOT = 1u << 0,        /* append: slot id outside the pool */
  MKV_DEVERR_BLOCK = 1u << 1,       /* gather/attention: block id outside the pool */
  MKV_DEVERR_TABLE = 1u << 2,       /* block table shorter than ceil(ctx/page_size) */
  MKV_DEVERR_COPY = 1u << 3,        /* copy_blocks: src or dst outside the pool */
  MKV_DEVERR_CTX = 1u << 4,         /* context length < 1 or > the max_ctx_len given */
  MKV_DEVERR_CHECKSUM = 1u << 5     /* wire import: a block's payload checksum differs */
};

/* decode_attention flags. */
enum {
  MKV_ATTN_ZERO_SINK = 1u << 0,  /* add the reference's phantom zero key/value:
                                    inference-model-qwen/src/model.rs:210-213 */
  MKV_ATTN_FORCE_VALU = 1u << 1, /* use the VALU kernel even where MFMA applies */
  MKV_ATTN_FORCE_MFMA = 1u << 2, /* fail unless the MFMA kernel applies */
  MKV_ATTN_PER_HEAD_LOADS = 1u << 3, /* planned MFMA path: one wave per KV head loads its
                                        own rows, instead of the workgroup loading whole
                                        token rows of every head (same results) */
  MKV_ATTN_CACHED_LOADS = 1u << 4     /* planned MFMA path: K/V loads through the caches
                                        instead of non-temporal. For batches whose tables
                                        share blocks (a radix-shared prefix: its blocks are
                                        re-read from the cache); slower for distinct blocks.
                                        Same results. */
};

/* qk_norm_rope_append flags. */
enum {
  MKV_PREP_PLAIN_Q = 1u << 0, /* d_q is [n][num_q_heads][head_dim] (no gate half) */
  MKV_PREP_NO_NORM = 1u << 1  /* skip the RMSNorm (RoPE and append only) */
};

typedef struct mkv_pool mkv_pool;

/* Pool descriptor. Extends the engine's ModelConfig
 * (inference-backend/src/config.rs:1-11: num_layers, num_kv_heads, head_dim)
 * with num_q_heads, which ModelConfig lacks, and the pool sizing of
 * EngineConfig (inference-engine/src/config.rs:3-17: num_kv_pages, page_size). */
typedef struct {
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t num_q_heads;  /* multiple of num_kv_heads */
  int32_t head_dim;     /* multiple of 8, at most 512 */
  int32_t page_size;    /* tokens per block; must be 16 */
  int32_t dtype;        /* mkv_dtype */
  int64_t num_blocks;   /* pages in the pool */
} mkv_pool_desc;

/* ---- pool lifecycle ------------------------------------------------------ */

/* Bytes of the pool: 2*L*blocks*page_size*Hkv*D*dtype_bytes.
 * Replaces KvCachePool::required_bytes (inference-engine/src/kv_pool.rs:58-68). */
MKV_API int mkv_pool_required_bytes(const mkv_pool_desc *desc, uint64_t *out_bytes);

/* Allocate the device pool on `device` (hipMalloc; contents uninitialised).
 * Replaces the device half of KvCachePool::new (kv_pool.rs:18-27) and the
 * design's KvBufferHandle (design/phase0-deliverable.md:1320-1332).
 * MKV_ERR_OUT_OF_MEMORY if HBM cannot hold it. */
MKV_API int mkv_pool_create(const mkv_pool_desc *desc, int device, mkv_pool **out_pool);
MKV_API int mkv_pool_destroy(mkv_pool *pool);
MKV_API int mkv_pool_get_desc(const mkv_pool *pool, mkv_pool_desc *out_desc);
/* Device base address and size of the pool buffer (for host read-back). */
MKV_API int mkv_pool_buffer(const mkv_pool *pool, void **out_dev_ptr, uint64_t *out_bytes);

/* Synchronise `stream`, then read and clear the device error word.
 * Returns MKV_ERR_DEVICE_INDEX if any bit was set (bits in *out_bits). */
MKV_API int mkv_pool_check(mkv_pool *pool, void *stream, uint32_t *out_bits);

/* Measurement hook (no counterpart in the reference: it lets a caller time
 * the decode step's dominant kernel alone with events). The next
 * mkv_decode_step, mkv_decode_attention_planned or (its suffix kernel)
 * mkv_decode_step_shared_prefix call on this pool records ev_start (a
 * hipEvent_t) on its stream right before its attention kernel and ev_end
 * right after it, before the split-K merge, then forgets both. NULL, NULL
 * forgets them now. */
MKV_API int mkv_pool_set_launch_events(mkv_pool *pool, void *ev_start, void *ev_end);

/* ---- data-plane operations ----------------------------------------------- */

/* Append num_tokens K/V rows into `layer`:
 *   pool[layer][K][s/ps][s%ps] = d_k[t],  pool[layer][V][s/ps][s%ps] = d_v[t],
 *   s = d_slot_mapping[t].
 * d_k, d_v: [num_tokens][num_kv_heads][head_dim] in the pool dtype.
 * Replaces the per-layer Tensor::cat append
 * (inference-model-qwen/src/model.rs:390-392). */
MKV_API int mkv_append(mkv_pool *pool, int32_t layer, const void *d_k, const void *d_v,
               const int32_t *d_slot_mapping, int32_t num_tokens, void *stream);

/* All layers in one launch: d_k, d_v are [num_layers][num_tokens][Hkv][D];
 * the same slot mapping applies to every layer. */
MKV_API int mkv_append_all_layers(mkv_pool *pool, const void *d_k, const void *d_v,
                          const int32_t *d_slot_mapping, int32_t num_tokens, void *stream);

/* Gather: for each sequence b, its first n_b = d_ctx_indptr[b+1]-d_ctx_indptr[b]
 * tokens, found through the block table
 * d_block_ids[d_block_indptr[b] .. d_block_indptr[b+1]), are written as
 * [num_kv_heads][n_b][head_dim] at element offset d_ctx_indptr[b]*Hkv*D of
 * d_out_k / d_out_v (the KVCacheState layout [batch, heads, seq, head_dim],
 * inference-model-common/src/lib.rs:5-8). max_ctx_len bounds every n_b;
 * out_capacity_tokens (tokens the outputs hold) bounds d_ctx_indptr[b+1]:
 * a sequence that would overflow is skipped and reported (MKV_DEVERR_CTX).
 * Implements the design's gather-then-attend copy
 * (design/phase0-deliverable.md:278; CSR kv_indptr/kv_indices,
 * design/rust-inference-engine-design.md:1505-1534). */
MKV_API int mkv_gather(mkv_pool *pool, int32_t layer, const int32_t *d_block_indptr,
                       const int32_t *d_block_ids, const int32_t *d_ctx_indptr, int32_t num_seqs,
                       int32_t max_ctx_len, void *d_out_k, void *d_out_v,
                       int64_t out_capacity_tokens, void *stream);

/* Copy whole blocks, all layers, K and V: pool[*][*][dst[i]] = pool[*][*][src[i]].
 * The result is defined when no block id is both a source and a destination
 * and destinations are distinct (mkv_validate_copy_pairs). Serves copy-on-write
 * of a shared partial block and the batched moves of pool compaction; the
 * reference has no counterpart (it aliases shared pages, prefill.rs:60-71). */
MKV_API int mkv_copy_blocks(mkv_pool *pool, const int32_t *d_src_blocks, const int32_t *d_dst_blocks,
                    int32_t num_pairs, void *stream);

/* Paged decode attention for one layer, one query row per sequence:
 *   O[b][h] = softmax(scale * Q[b][h] . K_b^T) . V_b
 * over the first d_ctx_lens[b] tokens of sequence b (block table CSR as in
 * mkv_gather), query head h reading KV head h / (num_q_heads/num_kv_heads).
 * d_q, d_o: [num_seqs][num_q_heads][head_dim] in the pool dtype; accumulation
 * is f32. max_ctx_len >= every d_ctx_lens[b] >= 1 sizes the launch.
 * split_tokens: context tokens per split-K partition (multiple of page_size),
 * 0 = chosen by the library. Workspace: device scratch of at least
 * mkv_decode_attention_workspace_size() bytes, or NULL to use a pool-owned
 * buffer (grown on demand). Replaces model.rs:394-416 (repeat_kv, q.k^T*scaling,
 * mask, softmax, .v). */
MKV_API int mkv_decode_attention(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                         const int32_t *d_block_indptr, const int32_t *d_block_ids,
                         const int32_t *d_ctx_lens, int32_t num_seqs, int32_t max_ctx_len,
                         float scale, uint32_t flags, int32_t split_tokens, void *d_workspace,
                         uint64_t workspace_bytes, void *stream);

MKV_API int mkv_decode_attention_workspace_size(const mkv_pool *pool, int32_t num_seqs,
                                        int32_t max_ctx_len, int32_t split_tokens,
                                        uint64_t *out_bytes);

/* mkv_decode_attention without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and results as mkv_decode_attention with a
 * caller workspace, except that the split-K partials live in a static device
 * array of MKV_STATIC_SCRATCH_BYTES that the library holds on each GPU it
 * runs on until the process ends (its address is looked up when the first
 * pool is created on that GPU). It calls no hipMalloc / hipFree. With
 * split_tokens = 0 the split is the library's choice, reduced until its
 * partials fit the array; an explicit split_tokens whose partials do not fit
 * is refused (MKV_ERR_INVALID_ARGUMENT). Every call on one GPU shares the
 * array: calls that overlap on one GPU (other streams or threads) race. */
#define MKV_STATIC_SCRATCH_BYTES (64ull << 20)
MKV_API int mkv_decode_attention_static(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                        const int32_t *d_block_indptr, const int32_t *d_block_ids,
                                        const int32_t *d_ctx_lens, int32_t num_seqs, int32_t max_ctx_len,
                                        float scale, uint32_t flags, int32_t split_tokens, void *stream);

/* ---- host metadata (the engine's u32 form) ------------------------------- */

/* mkv_append with a host slot mapping (slot = page * page_size + offset, as
 * the engine derives it from kv_pages: prefill.rs:72-81, scheduler.rs:42-57).
 * A mapping equal to the previous call's (same stream) is not uploaded
 * again. */
MKV_API int mkv_append_host(mkv_pool *pool, int32_t layer, const void *d_k, const void *d_v,
                            const uint32_t *h_slot_mapping, int32_t num_tokens, void *stream);
/* mkv_append_all_layers with a host slot mapping. */
MKV_API int mkv_append_all_layers_host(mkv_pool *pool, const void *d_k, const void *d_v,
                                       const uint32_t *h_slot_mapping, int32_t num_tokens, void *stream);
/* mkv_gather with host tables: sequence b's first h_ctx_lens[b] tokens
 * through table h_block_ids[h_block_indptr[b] ..), written at element offset
 * (sum of the earlier h_ctx_lens) * Hkv * D of the outputs. Tables equal to
 * the previous call's (same stream) are not uploaded again. */
MKV_API int mkv_gather_host(mkv_pool *pool, int32_t layer, const uint32_t *h_block_indptr,
                            const uint32_t *h_block_ids, const int32_t *h_ctx_lens, int32_t num_seqs,
                            void *d_out_k, void *d_out_v, int64_t out_capacity_tokens, void *stream);
/* mkv_copy_blocks with host pairs; the pairs are checked as
 * mkv_validate_copy_pairs does (distinct destinations, no block both a
 * source and a destination) before anything is launched. */
MKV_API int mkv_copy_blocks_host(mkv_pool *pool, const uint32_t *h_src_blocks, const uint32_t *h_dst_blocks,
                                 int32_t num_pairs, void *stream);
/* mkv_extend_attention with host metadata: sequence b has h_q_lens[b] new
 * tokens (its extend_len, request.rs:46-54; 0 <= q_len <= ctx) whose query
 * rows follow those of sequence b-1 in d_q / d_o, and h_ctx_lens[b] tokens
 * in its table (the chunk included). Metadata equal to the previous call's
 * (same stream) is not uploaded again. */
MKV_API int mkv_extend_attention_host(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                      const int32_t *h_q_lens, const int32_t *h_ctx_lens,
                                      const uint32_t *h_block_indptr, const uint32_t *h_block_ids,
                                      int32_t num_seqs, float scale, uint32_t flags, void *stream);
/* mkv_qk_norm_rope_append with host positions and slots. */
MKV_API int mkv_qk_norm_rope_append_host(mkv_pool *pool, int32_t layer, const void *d_q, const void *d_k,
                                         const void *d_v, const float *d_q_norm_w, const float *d_k_norm_w,
                                         const float *d_inv_freq, int32_t rotary_dim, float eps,
                                         const int32_t *h_positions, const uint32_t *h_slot_mapping,
                                         int32_t num_tokens, void *d_q_out, uint32_t flags, void *stream);
/* mkv_wire_export / mkv_wire_import with host block ids; the import's
 * destinations must be distinct (checked). */
MKV_API int mkv_wire_export_host(mkv_pool *pool, const uint32_t *h_block_ids, int32_t num_blocks,
                                 int32_t layer_begin, int32_t num_layers, void *d_payload, uint64_t *d_checksums,
                                 void *stream);
MKV_API int mkv_wire_import_host(mkv_pool *pool, const uint32_t *h_block_ids, int32_t num_blocks,
                                 int32_t layer_begin, int32_t num_layers, const void *d_payload,
                                 const uint64_t *d_expected, uint64_t *d_checksums, void *stream);

/* ---- planned decode (production path) ----------------------------------- */

/* A decode plan is the work decomposition of one engine step, built on the
 * host from the host-side context lengths (the scheduler has them: it is the
 * Batch it assembles, inference-engine/src/scheduler.rs:29-77) and uploaded
 * once; every layer's attention call of that step reuses it. The
 * concatenation of all sequences' blocks is cut into `pieces` equal runs,
 * one workgroup each, so the work per workgroup does not depend on how
 * ragged the contexts are. The plan owns its metadata and split-K scratch. */
typedef struct mkv_decode_plan mkv_decode_plan;

MKV_API int mkv_decode_plan_create(mkv_pool *pool, mkv_decode_plan **out_plan);
MKV_API int mkv_decode_plan_destroy(mkv_decode_plan *plan);
/* h_ctx_lens: host array, tokens each sequence attends (>= 1).
 * pieces: 0 = chosen by the library. Uploads asynchronously on `stream`.
 * A plan built this way has no tables: its decode calls pass device tables. */
MKV_API int mkv_decode_plan_build(mkv_decode_plan *plan, const int32_t *h_ctx_lens,
                                  int32_t num_seqs, int32_t pieces, void *stream);
/* The engine's one call per step: mkv_decode_plan_build plus the batch's
 * page tables as host CSR (u32 indptr[num_seqs+1], u32 ids), validated
 * against the pool and copied into the plan (uploaded on `stream` with the
 * plan). The step's decode calls then pass NULL tables and read the plan's.
 * A later build replaces the tables; the calls already enqueued keep the
 * ones they were enqueued with only if they run first on the same stream,
 * so rebuild a plan on the stream that uses it. */
MKV_API int mkv_decode_plan_build_tables(mkv_decode_plan *plan, const int32_t *h_ctx_lens,
                                         const uint32_t *h_block_indptr, const uint32_t *h_block_ids,
                                         int32_t num_seqs, int32_t pieces, void *stream);
MKV_API int mkv_decode_plan_info(const mkv_decode_plan *plan, int32_t *out_pieces,
                                 int32_t *out_blocks_per_piece, int32_t *out_merge_seqs);
/* mkv_decode_attention over the plan's sequences and context lengths.
 * Tables: d_block_indptr / d_block_ids (device, read on every call, so a
 * table rewritten in place between calls is seen by the next one), or both
 * NULL for the tables given to mkv_decode_plan_build_tables. */
MKV_API int mkv_decode_attention_planned(mkv_pool *pool, const mkv_decode_plan *plan,
                                         int32_t layer, const void *d_q, void *d_o,
                                         const int32_t *d_block_indptr,
                                         const int32_t *d_block_ids, float scale,
                                         uint32_t flags, void *stream);
/* One decode step of one layer in one launch: for every sequence b, write
 * d_k_new[b], d_v_new[b] ([num_seqs][num_kv_heads][head_dim]) at position
 * ctx_b - 1 (its slot from its block table), then attend over ctx_b tokens.
 * Equal to mkv_append at those slots followed by
 * mkv_decode_attention_planned (tables as there: device, or both NULL for
 * the plan's). Replaces model.rs:390-416 for one layer. */
MKV_API int mkv_decode_step(mkv_pool *pool, const mkv_decode_plan *plan, int32_t layer,
                            const void *d_k_new, const void *d_v_new, const void *d_q, void *d_o,
                            const int32_t *d_block_indptr, const int32_t *d_block_ids,
                            float scale, uint32_t flags, void *stream);
/* mkv_decode_step that also writes the layer's block-table gather, the
 * grown KVCacheState of model.rs:390-392 (the step's new row included):
 * what mkv_gather writes for the plan's sequences and contexts, sequence b's
 * [num_kv_heads][ctx_b][head_dim] at element offset (ctx_0 + ... +
 * ctx_{b-1}) * num_kv_heads * head_dim of d_out_k / d_out_v (capacity
 * out_capacity_tokens tokens, 16-byte aligned). On the per-head kernel (f32
 * pools, and bf16 ones the MFMA kernels do not take) the attention kernel
 * stores the rows as it reads them; after the MFMA kernels the gather
 * kernel follows on the same stream. Not for suffix plans. */
MKV_API int mkv_decode_step_gather(mkv_pool *pool, const mkv_decode_plan *plan, int32_t layer,
                                   const void *d_k_new, const void *d_v_new, const void *d_q, void *d_o,
                                   const int32_t *d_block_indptr, const int32_t *d_block_ids,
                                   void *d_out_k, void *d_out_v, int64_t out_capacity_tokens,
                                   float scale, uint32_t flags, void *stream);

/* ---- decode over a shared prefix ------------------------------------------ */

/* A step whose sequences all share one prefix of full blocks, as radix
 * sharing hands them out (inference-engine/src/radix_cache.rs:64-117 returns
 * the same pages to every request that matched the prefix). There is no
 * counterpart in the reference: it keeps one contiguous cache per request
 * and attends over the prefix again for each (model.rs:390-416). Here the
 * prefix's K/V are read once for all sequences and its attention runs on
 * MFMA tiles. Sequence b attends the prefix's 16 * prefix_blocks tokens
 * followed by its suffix of suffix_len_b tokens.
 *
 * mkv_decode_plan_build_suffixes: as mkv_decode_plan_build, over the suffix
 * lengths (>= 1: the appended token is in the suffix). A plan built this way
 * stores every sequence's result as partials for the step below.
 *
 * mkv_decode_plan_build_shared_prefix: the same with the host tables of the
 * suffixes and the prefix's u32 block ids, copied into the plan.
 *
 * mkv_decode_step_shared_prefix: mkv_decode_step over prefix + suffix.
 * d_prefix_ids: the prefix's prefix_blocks block ids (device), or NULL for
 * the plan's. The tables d_block_indptr / d_block_ids (device, or both NULL
 * for the plan's) hold each sequence's suffix blocks only;
 * d_k_new / d_v_new (both or neither) go at suffix position suffix_len_b - 1.
 * Three launches: the prefix over all queries (f32 partials per key range in
 * the pool-owned workspace, grown on demand as for mkv_extend_attention),
 * the suffixes through the plan, and their merge. Where a workgroup of the
 * prefix fits beside one of the suffixes on every compute unit (the pool's
 * geometry decides; Qwen2.5-7B heads do), a plan built with pieces = 0 cuts
 * one suffix piece per compute unit and the step runs the prefix on a
 * second HIP stream that the pool creates on first use: forked from
 * `stream` at entry and joined back into it before the merge, so work
 * enqueued on `stream` after the call still follows the whole step. Calls
 * on one pool must not overlap on different streams (they share the
 * workspace and that second stream). bf16 pools, head_dim
 * 64/128/256, at most 16 query heads per KV head. Same result as
 * mkv_decode_step over tables prefix + suffix, within the attention
 * tolerance (the partials merge in another order). Flags: MKV_ATTN_ZERO_SINK. */
MKV_API int mkv_decode_plan_build_suffixes(mkv_decode_plan *plan, const int32_t *h_suffix_lens,
                                           int32_t num_seqs, int32_t pieces, void *stream);
MKV_API int mkv_decode_plan_build_shared_prefix(mkv_decode_plan *plan, const uint32_t *h_prefix_ids,
                                                int32_t prefix_blocks, const int32_t *h_suffix_lens,
                                                const uint32_t *h_block_indptr, const uint32_t *h_block_ids,
                                                int32_t num_seqs, int32_t pieces, void *stream);
MKV_API int mkv_decode_step_shared_prefix(mkv_pool *pool, const mkv_decode_plan *plan,
                                          int32_t layer, const void *d_k_new, const void *d_v_new,
                                          const void *d_q, void *d_o, const int32_t *d_prefix_ids,
                                          int32_t prefix_blocks, const int32_t *d_block_indptr,
                                          const int32_t *d_block_ids, float scale, uint32_t flags,
                                          void *stream);

/* ---- extend (chunked prefill) attention ----------------------------------- */

/* Causal attention of each sequence's newest tokens over its whole cache:
 * sequence b has n_b = d_q_indptr[b+1] - d_q_indptr[b] query tokens at
 * positions [ctx_b - n_b, ctx_b) (ctx_b = d_ctx_lens[b], the chunk's K/V
 * already appended with mkv_append); the query at position p attends keys
 * 0..p. d_q, d_o: [d_q_indptr[num_seqs]][num_q_heads][head_dim].
 * max_q_len / max_ctx_len bound n_b / ctx_b (a larger ctx_b is skipped and
 * reported, MKV_DEVERR_CTX). Any pool: bf16 pools with head_dim 64/128/256
 * and at most 16 query heads per KV head run MFMA query tiles; other pools
 * (f32, head_dim 32, larger groups) run one decode segment per query token.
 * When the MFMA tiles would leave the device's resident workgroup slots
 * empty (few short chunks over long contexts), each key range is split in up
 * to 4 and the f32 partials are merged by a second launch; they use the
 * pool-owned workspace shared with mkv_decode_attention (grown on demand:
 * that call synchronises the stream once, and such calls on one pool must
 * not run concurrently on different streams).
 * Flags: MKV_ATTN_ZERO_SINK.
 * Replaces the seq_q > 1 path of inference-model-qwen/src/model.rs:410-416
 * with its causal mask (model.rs:542-555), for the chunks scheduled by
 * inference-engine/src/prefill.rs:99-114. d_q / d_o are in the pool dtype. */
MKV_API int mkv_extend_attention(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                 const int32_t *d_q_indptr, const int32_t *d_block_indptr,
                                 const int32_t *d_block_ids, const int32_t *d_ctx_lens, int32_t num_seqs,
                                 int32_t max_q_len, int32_t max_ctx_len, float scale, uint32_t flags,
                                 void *stream);

/* ---- fused pre-attention step --------------------------------------------- */

/* For each token t of one layer: RMSNorm of every q head and k head,
 *   x * (mean(x^2) + eps)^-1/2 * (1 + w)   (w = d_q_norm_w or d_k_norm_w, [head_dim] f32),
 * then NeoX RoPE on dims [0, rotary_dim) at position d_positions[t]: for
 * i < rotary_dim/2, angle a = pos * d_inv_freq[i],
 *   x[i] -> x[i]*cos a - x[i+half]*sin a,  x[i+half] -> x[i+half]*cos a + x[i]*sin a,
 * dims >= rotary_dim unchanged. The prepared k row and the unchanged v row are
 * appended at slot d_slot_mapping[t] (as mkv_append); the prepared q rows go
 * to d_q_out [num_tokens][num_q_heads][head_dim]. All in the pool dtype,
 * computed in f32 with one rounding per output element.
 * d_q: [num_tokens][num_q_heads][2][head_dim] (q then gate, the q_proj output)
 * or, with MKV_PREP_PLAIN_Q, [num_tokens][num_q_heads][head_dim].
 * d_k, d_v: [num_tokens][num_kv_heads][head_dim]. d_inv_freq: [rotary_dim/2]
 * f32, the reference's 1 / theta^(2i/rotary_dim). rotary_dim must be a
 * multiple of 2*max(1, head_dim/64); head_dim 32/64/128/256.
 * With MKV_PREP_NO_NORM the weights may be NULL and eps is ignored.
 * Replaces, for one layer, inference-model-qwen/src/model.rs:371-392:
 * the q slice of the gated q_proj (:371-374), RmsNorm::forward4 (:104-108),
 * apply_rope (:508-540) on q and k, and the cache append (:390-392). */
MKV_API int mkv_qk_norm_rope_append(mkv_pool *pool, int32_t layer, const void *d_q, const void *d_k,
                                    const void *d_v, const float *d_q_norm_w, const float *d_k_norm_w,
                                    const float *d_inv_freq, int32_t rotary_dim, float eps,
                                    const int32_t *d_positions, const int32_t *d_slot_mapping,
                                    int32_t num_tokens, void *d_q_out, uint32_t flags, void *stream);

/* ---- KV block wire format --------------------------------------------------- */

/* Blocks leave and enter a pool as a payload of
 *   [num_blocks][num_layers][2 (K, V)][page_size][num_kv_heads][head_dim]
 * (pool dtype, block-major: one block's state is contiguous) with one u64
 * checksum per block: over the block's payload as little-endian u64 words
 * w_0 .. w_{m-1},
 *   sum64 = sum_j mix(w_j + (j + 1) * 0x9E3779B97F4A7C15)  (mod 2^64),
 *   mix(z): z = (z ^ z>>30) * 0xBF58476D1CE4E5B9; z = (z ^ z>>27) * 0x94D049BB133111EB; z ^ z>>31.
 * A file or message is: mkv_wire_header (64 bytes) | num_blocks checksums
 * (u64) | zero padding | payload at header.payload_offset (a multiple of
 * 4096). All fields little-endian.
 * The reference hands pages between workers as indices into one pool
 * (KvHandoff { request_id, kv_pages, cached_len },
 * design/phase2b-deliverable.md:272-289) and plans per-layer KV files for
 * SSD offload (KvOffloadManager, design/phase1-deliverable.md:253-339); this
 * is the byte form of both: a handoff carries all layers of a request's
 * pages, an offload chunk one layer (num_layers = 1). */
#define MKV_WIRE_MAGIC 0x57564B4Du /* "MKVW" */
#define MKV_WIRE_VERSION 1u

typedef struct mkv_wire_header {
  uint32_t magic;          /* MKV_WIRE_MAGIC */
  uint16_t version;        /* MKV_WIRE_VERSION */
  uint16_t dtype;          /* MKV_DTYPE_* */
  int32_t page_size;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t layer_begin;     /* first layer carried */
  int32_t num_layers;      /* layers carried */
  int32_t num_blocks;
  int64_t cached_len;      /* tokens the blocks hold (KvHandoff.cached_len) */
  uint64_t block_bytes;    /* payload bytes per block */
  uint64_t payload_offset; /* byte offset of the payload from the header's start */
  uint64_t reserved;       /* 0 */
} mkv_wire_header;

/* Copy layers [layer_begin, layer_begin + num_layers) of blocks
 * d_block_ids[0..num_blocks) into d_payload (num_blocks * block_bytes) and
 * their checksums into d_checksums[num_blocks]. An id outside the pool is
 * skipped and reported (MKV_DEVERR_BLOCK). At most 65535 blocks per call.
 * No reference counterpart (see above); the read side of a handoff or an
 * offload write-back. */
MKV_API int mkv_wire_export(mkv_pool *pool, const int32_t *d_block_ids, int32_t num_blocks,
                            int32_t layer_begin, int32_t num_layers, void *d_payload, uint64_t *d_checksums,
                            void *stream);
/* Copy d_payload into blocks d_block_ids (distinct; see
 * mkv_validate_copy_pairs) and write the checksums of the payload as
 * received to d_checksums. With d_expected non-NULL, a block whose checksum
 * differs sets MKV_DEVERR_CHECKSUM (its bytes are still written: import into
 * fresh blocks and release them if mkv_pool_check reports it). */
MKV_API int mkv_wire_import(mkv_pool *pool, const int32_t *d_block_ids, int32_t num_blocks,
                            int32_t layer_begin, int32_t num_layers, const void *d_payload,
                            const uint64_t *d_expected, uint64_t *d_checksums, void *stream);
/* Fill a header for a payload of this pool (pure CPU). */
MKV_API int mkv_wire_header_init(const mkv_pool_desc *desc, int32_t layer_begin, int32_t num_layers,
                                 int32_t num_blocks, int64_t cached_len, mkv_wire_header *out);
/* MKV_OK if the header is a version this library reads and its geometry
 * fits the pool (pure CPU). */
MKV_API int mkv_wire_header_check(const mkv_pool_desc *desc, const mkv_wire_header *header);

/* ---- host-side validation (pure CPU; no device access) ------------------- */

/* 0 <= slot < num_blocks*page_size for every slot. */
MKV_API int mkv_validate_slots(const mkv_pool_desc *desc, const int32_t *slots, int32_t n);
/* indptr monotone, ids in range, table b holds >= ceil(ctx_b/page_size) ids,
 * 1 <= ctx_b <= max_ctx_len. ctx_lens may be NULL (tables only). */
MKV_API int mkv_validate_block_tables(const mkv_pool_desc *desc, const int32_t *indptr,
                              const int32_t *ids, const int32_t *ctx_lens, int32_t num_seqs,
                              int32_t max_ctx_len);
/* ids in range, destinations distinct, no id both source and destination. */
MKV_API int mkv_validate_copy_pairs(const mkv_pool_desc *desc, const int32_t *src, const int32_t *dst,
                            int32_t n);

/* ---- device buffers (the backend's device-buffer type) ------------------- */

/* hipMalloc on `device` (the backend's device-buffer allocation).
 * MKV_ERR_NO_DEVICE without a HIP device, MKV_ERR_INVALID_ARGUMENT for a
 * device index out of range or a NULL out pointer, MKV_ERR_OUT_OF_MEMORY. A
 * HIP failure returned as a status leaves no HIP error behind for the
 * caller's next check (true of every entry point). */
MKV_API int mkv_buffer_alloc(int device, uint64_t bytes, void **out_dev_ptr);
MKV_API int mkv_buffer_free(void *dev_ptr);
/* Host -> device on `stream`; the host buffer must stay valid until the
 * stream reaches this point. */
MKV_API int mkv_memcpy_h2d(void *d_dst, const void *h_src, uint64_t bytes, void *stream);
/* Device -> host on `stream`, synchronous on return. */
MKV_API int mkv_memcpy_d2h(void *h_dst, const void *d_src, uint64_t bytes, void *stream);
MKV_API int mkv_stream_synchronize(void *stream);

/* ---- diagnostics --------------------------------------------------------- */

MKV_API const char *mkv_last_error(void);
/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
MKV_API int mkv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MITTEN_KV_H */
