//! Raw FFI of `libmitten_kv.so`, the device library of the paged KV path
//! (`include/mitten_kv.h`, one declaration per exported function, same
//! order and parameter types). The engine-facing safe layer is the
//! `mitten-kv` crate; nothing here allocates or checks anything.
//!
//! Every function returns an `mkv_status` (`MKV_OK` = 0); the message of
//! the last failure on the calling thread is `mkv_last_error()`.
#![allow(non_camel_case_types)]
use std::ffi::{c_char, c_void};

pub const MKV_OK: i32 = 0;
pub const MKV_ERR_INVALID_ARGUMENT: i32 = 1;
pub const MKV_ERR_OUT_OF_MEMORY: i32 = 2;
pub const MKV_ERR_HIP: i32 = 3;
pub const MKV_ERR_DEVICE_INDEX: i32 = 4;
pub const MKV_ERR_NO_DEVICE: i32 = 5;
pub const MKV_DTYPE_F32: i32 = 0;
pub const MKV_DTYPE_BF16: i32 = 1;
pub const MKV_DEVERR_SLOT: u32 = 1;
pub const MKV_DEVERR_BLOCK: u32 = 2;
pub const MKV_DEVERR_TABLE: u32 = 4;
pub const MKV_DEVERR_COPY: u32 = 8;
pub const MKV_DEVERR_CTX: u32 = 16;
pub const MKV_DEVERR_CHECKSUM: u32 = 32;
pub const MKV_ATTN_ZERO_SINK: u32 = 1;
pub const MKV_ATTN_FORCE_VALU: u32 = 2;
pub const MKV_ATTN_FORCE_MFMA: u32 = 4;
pub const MKV_ATTN_PER_HEAD_LOADS: u32 = 8;
pub const MKV_ATTN_CACHED_LOADS: u32 = 16;
pub const MKV_PREP_PLAIN_Q: u32 = 1;
pub const MKV_PREP_NO_NORM: u32 = 2;
pub const MKV_WIRE_MAGIC: u32 = 0x57564B4D;
pub const MKV_WIRE_VERSION: u32 = 1;
pub const MKV_STATIC_SCRATCH_BYTES: u64 = 64 << 20;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mkv_pool_desc {
    pub num_layers: i32,
    pub num_kv_heads: i32,
    pub num_q_heads: i32,
    pub head_dim: i32,
    pub page_size: i32,
    pub dtype: i32,
    pub num_blocks: i64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct mkv_wire_header {
    pub magic: u32, pub version: u16, pub dtype: u16,
    pub page_size: i32, pub num_kv_heads: i32, pub head_dim: i32,
    pub layer_begin: i32, pub num_layers: i32, pub num_blocks: i32,
    pub cached_len: i64, pub block_bytes: u64, pub payload_offset: u64, pub reserved: u64,
}
#[repr(C)] pub struct mkv_pool { _p: [u8; 0] }
#[repr(C)] pub struct mkv_decode_plan { _p: [u8; 0] }
pub type hipStream_t = *mut c_void;

extern "C" {
    pub fn mkv_pool_required_bytes(desc: *const mkv_pool_desc, out_bytes: *mut u64) -> i32;
    pub fn mkv_pool_create(desc: *const mkv_pool_desc, device: i32, out_pool: *mut *mut mkv_pool) -> i32;
    pub fn mkv_pool_destroy(pool: *mut mkv_pool) -> i32;
    pub fn mkv_pool_get_desc(pool: *const mkv_pool, out_desc: *mut mkv_pool_desc) -> i32;
    pub fn mkv_pool_buffer(pool: *const mkv_pool, out_dev_ptr: *mut *mut c_void, out_bytes: *mut u64) -> i32;
    pub fn mkv_pool_check(pool: *mut mkv_pool, stream: hipStream_t, out_bits: *mut u32) -> i32;
    pub fn mkv_pool_set_launch_events(pool: *mut mkv_pool, ev_start: *mut c_void, ev_end: *mut c_void) -> i32;
    pub fn mkv_append(pool: *mut mkv_pool, layer: i32, d_k: *const c_void, d_v: *const c_void,
                      d_slot_mapping: *const i32, num_tokens: i32, stream: hipStream_t) -> i32;
    pub fn mkv_append_all_layers(pool: *mut mkv_pool, d_k: *const c_void, d_v: *const c_void,
                                 d_slot_mapping: *const i32, num_tokens: i32, stream: hipStream_t) -> i32;
    pub fn mkv_gather(pool: *mut mkv_pool, layer: i32, d_block_indptr: *const i32, d_block_ids: *const i32,
                      d_ctx_indptr: *const i32, num_seqs: i32, max_ctx_len: i32, d_out_k: *mut c_void,
                      d_out_v: *mut c_void, out_capacity_tokens: i64, stream: hipStream_t) -> i32;
    pub fn mkv_copy_blocks(pool: *mut mkv_pool, d_src_blocks: *const i32, d_dst_blocks: *const i32,
                           num_pairs: i32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_attention(pool: *mut mkv_pool, layer: i32, d_q: *const c_void, d_o: *mut c_void,
                                d_block_indptr: *const i32, d_block_ids: *const i32, d_ctx_lens: *const i32,
                                num_seqs: i32, max_ctx_len: i32, scale: f32, flags: u32, split_tokens: i32,
                                d_workspace: *mut c_void, workspace_bytes: u64, stream: hipStream_t) -> i32;
    pub fn mkv_decode_attention_workspace_size(pool: *const mkv_pool, num_seqs: i32, max_ctx_len: i32,
                                               split_tokens: i32, out_bytes: *mut u64) -> i32;
    pub fn mkv_decode_attention_static(pool: *mut mkv_pool, layer: i32, d_q: *const c_void, d_o: *mut c_void,
                                       d_block_indptr: *const i32, d_block_ids: *const i32,
                                       d_ctx_lens: *const i32, num_seqs: i32, max_ctx_len: i32, scale: f32,
                                       flags: u32, split_tokens: i32, stream: hipStream_t) -> i32;
    pub fn mkv_append_host(pool: *mut mkv_pool, layer: i32, d_k: *const c_void, d_v: *const c_void,
                           h_slot_mapping: *const u32, num_tokens: i32, stream: hipStream_t) -> i32;
    pub fn mkv_append_all_layers_host(pool: *mut mkv_pool, d_k: *const c_void, d_v: *const c_void,
                                      h_slot_mapping: *const u32, num_tokens: i32,
                                      stream: hipStream_t) -> i32;
    pub fn mkv_gather_host(pool: *mut mkv_pool, layer: i32, h_block_indptr: *const u32,
                           h_block_ids: *const u32, h_ctx_lens: *const i32, num_seqs: i32,
                           d_out_k: *mut c_void, d_out_v: *mut c_void, out_capacity_tokens: i64,
                           stream: hipStream_t) -> i32;
    pub fn mkv_copy_blocks_host(pool: *mut mkv_pool, h_src_blocks: *const u32, h_dst_blocks: *const u32,
                                num_pairs: i32, stream: hipStream_t) -> i32;
    pub fn mkv_extend_attention_host(pool: *mut mkv_pool, layer: i32, d_q: *const c_void, d_o: *mut c_void,
                                     h_q_lens: *const i32, h_ctx_lens: *const i32,
                                     h_block_indptr: *const u32, h_block_ids: *const u32, num_seqs: i32,
                                     scale: f32, flags: u32, stream: hipStream_t) -> i32;
    pub fn mkv_qk_norm_rope_append_host(pool: *mut mkv_pool, layer: i32, d_q: *const c_void,
                                        d_k: *const c_void, d_v: *const c_void, d_q_norm_w: *const f32,
                                        d_k_norm_w: *const f32, d_inv_freq: *const f32, rotary_dim: i32,
                                        eps: f32, h_positions: *const i32, h_slot_mapping: *const u32,
                                        num_tokens: i32, d_q_out: *mut c_void, flags: u32,
                                        stream: hipStream_t) -> i32;
    pub fn mkv_wire_export_host(pool: *mut mkv_pool, h_block_ids: *const u32, num_blocks: i32,
                                layer_begin: i32, num_layers: i32, d_payload: *mut c_void,
                                d_checksums: *mut u64, stream: hipStream_t) -> i32;
    pub fn mkv_wire_import_host(pool: *mut mkv_pool, h_block_ids: *const u32, num_blocks: i32,
                                layer_begin: i32, num_layers: i32, d_payload: *const c_void,
                                d_expected: *const u64, d_checksums: *mut u64, stream: hipStream_t) -> i32;
    pub fn mkv_decode_plan_create(pool: *mut mkv_pool, out_plan: *mut *mut mkv_decode_plan) -> i32;
    pub fn mkv_decode_plan_destroy(plan: *mut mkv_decode_plan) -> i32;
    pub fn mkv_decode_plan_build(plan: *mut mkv_decode_plan, h_ctx_lens: *const i32, num_seqs: i32,
                                 pieces: i32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_plan_build_tables(plan: *mut mkv_decode_plan, h_ctx_lens: *const i32,
                                        h_block_indptr: *const u32, h_block_ids: *const u32, num_seqs: i32,
                                        pieces: i32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_plan_info(plan: *const mkv_decode_plan, out_pieces: *mut i32,
                                out_blocks_per_piece: *mut i32, out_merge_seqs: *mut i32) -> i32;
    pub fn mkv_decode_attention_planned(pool: *mut mkv_pool, plan: *const mkv_decode_plan, layer: i32,
                                        d_q: *const c_void, d_o: *mut c_void, d_block_indptr: *const i32,
                                        d_block_ids: *const i32, scale: f32, flags: u32,
                                        stream: hipStream_t) -> i32;
    pub fn mkv_decode_step(pool: *mut mkv_pool, plan: *const mkv_decode_plan, layer: i32,
                           d_k_new: *const c_void, d_v_new: *const c_void, d_q: *const c_void,
                           d_o: *mut c_void, d_block_indptr: *const i32, d_block_ids: *const i32, scale: f32,
                           flags: u32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_step_gather(pool: *mut mkv_pool, plan: *const mkv_decode_plan, layer: i32,
                                  d_k_new: *const c_void, d_v_new: *const c_void, d_q: *const c_void,
                                  d_o: *mut c_void, d_block_indptr: *const i32, d_block_ids: *const i32,
                                  d_out_k: *mut c_void, d_out_v: *mut c_void, out_capacity_tokens: i64,
                                  scale: f32, flags: u32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_plan_build_suffixes(plan: *mut mkv_decode_plan, h_suffix_lens: *const i32,
                                          num_seqs: i32, pieces: i32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_plan_build_shared_prefix(plan: *mut mkv_decode_plan, h_prefix_ids: *const u32,
                                               prefix_blocks: i32, h_suffix_lens: *const i32,
                                               h_block_indptr: *const u32, h_block_ids: *const u32,
                                               num_seqs: i32, pieces: i32, stream: hipStream_t) -> i32;
    pub fn mkv_decode_step_shared_prefix(pool: *mut mkv_pool, plan: *const mkv_decode_plan, layer: i32,
                                         d_k_new: *const c_void, d_v_new: *const c_void, d_q: *const c_void,
                                         d_o: *mut c_void, d_prefix_ids: *const i32, prefix_blocks: i32,
                                         d_block_indptr: *const i32, d_block_ids: *const i32, scale: f32,
                                         flags: u32, stream: hipStream_t) -> i32;
    pub fn mkv_extend_attention(pool: *mut mkv_pool, layer: i32, d_q: *const c_void, d_o: *mut c_void,
                                d_q_indptr: *const i32, d_block_indptr: *const i32, d_block_ids: *const i32,
                                d_ctx_lens: *const i32, num_seqs: i32, max_q_len: i32, max_ctx_len: i32,
                                scale: f32, flags: u32, stream: hipStream_t) -> i32;
    pub fn mkv_qk_norm_rope_append(pool: *mut mkv_pool, layer: i32, d_q: *const c_void, d_k: *const c_void,
                                   d_v: *const c_void, d_q_norm_w: *const f32, d_k_norm_w: *const f32,
                                   d_inv_freq: *const f32, rotary_dim: i32, eps: f32,
                                   d_positions: *const i32, d_slot_mapping: *const i32, num_tokens: i32,
                                   d_q_out: *mut c_void, flags: u32, stream: hipStream_t) -> i32;
    pub fn mkv_wire_export(pool: *mut mkv_pool, d_block_ids: *const i32, num_blocks: i32, layer_begin: i32,
                           num_layers: i32, d_payload: *mut c_void, d_checksums: *mut u64,
                           stream: hipStream_t) -> i32;
    pub fn mkv_wire_import(pool: *mut mkv_pool, d_block_ids: *const i32, num_blocks: i32, layer_begin: i32,
                           num_layers: i32, d_payload: *const c_void, d_expected: *const u64,
                           d_checksums: *mut u64, stream: hipStream_t) -> i32;
    pub fn mkv_wire_header_init(desc: *const mkv_pool_desc, layer_begin: i32, num_layers: i32,
                                num_blocks: i32, cached_len: i64, out: *mut mkv_wire_header) -> i32;
    pub fn mkv_wire_header_check(desc: *const mkv_pool_desc, header: *const mkv_wire_header) -> i32;
    pub fn mkv_validate_slots(desc: *const mkv_pool_desc, slots: *const i32, n: i32) -> i32;
    pub fn mkv_validate_block_tables(desc: *const mkv_pool_desc, indptr: *const i32, ids: *const i32,
                                     ctx_lens: *const i32, num_seqs: i32, max_ctx_len: i32) -> i32;
    pub fn mkv_validate_copy_pairs(desc: *const mkv_pool_desc, src: *const i32, dst: *const i32,
                                   n: i32) -> i32;
    pub fn mkv_buffer_alloc(device: i32, bytes: u64, out_dev_ptr: *mut *mut c_void) -> i32;
    pub fn mkv_buffer_free(dev_ptr: *mut c_void) -> i32;
    pub fn mkv_memcpy_h2d(d_dst: *mut c_void, h_src: *const c_void, bytes: u64, stream: hipStream_t) -> i32;
    pub fn mkv_memcpy_d2h(h_dst: *mut c_void, d_src: *const c_void, bytes: u64, stream: hipStream_t) -> i32;
    pub fn mkv_stream_synchronize(stream: hipStream_t) -> i32;
    pub fn mkv_last_error() -> *const c_char;
    pub fn mkv_version() -> i32;
}
