//! The backend's device KV pool: the "device-buffer type" of the paged path.
//!
//! The engine keeps page metadata on the host; the KV bytes live in one HBM
//! allocation owned here (`design/phase0-deliverable.md:1320-1332`), laid out
//! `[layer][K|V][block][16 tokens][kv head][head dim]`
//! (`design/rust-inference-engine-design.md:1385`). Owned by the GPU thread:
//! no call blocks except `check` and `synchronize`, and calls are ordered by
//! the stream they are given.

use crate::error::check;
use inference_backend::{EngineError, ModelConfig};
use mitten_kv_sys as sys;
use std::ffi::c_void;
use std::ptr;

/// Tokens per block (`inference-engine/src/kv_pool.rs`'s page size, 16 in
/// the reference configuration `design/phase2b-deliverable.md:960-962`).
pub const PAGE_SIZE: usize = 16;

/// A HIP stream handle; null is the device's default stream.
pub type Stream = sys::hipStream_t;

#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum KvDtype {
    F32,
    Bf16,
}

impl KvDtype {
    pub fn bytes(self) -> usize {
        match self {
            KvDtype::F32 => 4,
            KvDtype::Bf16 => 2,
        }
    }
    fn raw(self) -> i32 {
        match self {
            KvDtype::F32 => sys::MKV_DTYPE_F32,
            KvDtype::Bf16 => sys::MKV_DTYPE_BF16,
        }
    }
}

/// The pool's shape: the model's attention geometry and the block count.
#[derive(Clone, Copy, Debug)]
pub struct PoolGeometry {
    pub num_layers: usize,
    pub num_kv_heads: usize,
    pub num_q_heads: usize,
    pub head_dim: usize,
    pub num_blocks: usize,
    pub dtype: KvDtype,
}

impl PoolGeometry {
    /// From the engine's model configuration (`inference-backend/src/config.rs`),
    /// which carries no query-head count: the model crate supplies it.
    pub fn from_model(cfg: &ModelConfig, num_q_heads: usize, num_blocks: usize, dtype: KvDtype) -> Self {
        Self {
            num_layers: cfg.num_layers,
            num_kv_heads: cfg.num_kv_heads,
            num_q_heads,
            head_dim: cfg.head_dim,
            num_blocks,
            dtype,
        }
    }

    fn desc(&self) -> sys::mkv_pool_desc {
        sys::mkv_pool_desc {
            num_layers: self.num_layers as i32,
            num_kv_heads: self.num_kv_heads as i32,
            num_q_heads: self.num_q_heads as i32,
            head_dim: self.head_dim as i32,
            page_size: PAGE_SIZE as i32,
            dtype: self.dtype.raw(),
            num_blocks: self.num_blocks as i64,
        }
    }

    /// Bytes of the pool: `KvCachePool::required_bytes` (`kv_pool.rs:58-68`).
    pub fn required_bytes(&self) -> Result<u64, EngineError> {
        let mut out = 0u64;
        check(unsafe { sys::mkv_pool_required_bytes(&self.desc(), &mut out) })?;
        Ok(out)
    }

    /// Blocks that `bytes` of HBM hold at this geometry (200e9 bytes hold
    /// 217,982 Qwen2.5-7B blocks).
    pub fn blocks_for_bytes(&self, bytes: u64) -> usize {
        let per_block =
            (2 * self.num_layers * PAGE_SIZE * self.num_kv_heads * self.head_dim * self.dtype.bytes()) as u64;
        (bytes / per_block) as usize
    }

    /// Bytes of one token row of one layer's K (or V): every KV head.
    pub fn kv_row_bytes(&self) -> usize {
        self.num_kv_heads * self.head_dim * self.dtype.bytes()
    }

    /// Bytes of one token row of a query (or attention output).
    pub fn q_row_bytes(&self) -> usize {
        self.num_q_heads * self.head_dim * self.dtype.bytes()
    }

    /// Whether `mkv_decode_step_shared_prefix` takes this geometry: bf16 KV
    /// on the MFMA kernels (head_dim 64, 128 or 256, at most 16 query heads
    /// per KV head).
    pub fn shared_prefix_supported(&self) -> bool {
        self.dtype == KvDtype::Bf16
            && matches!(self.head_dim, 64 | 128 | 256)
            && self.num_q_heads <= 16 * self.num_kv_heads
    }
}

/// Page tables in the C ABI's CSR form (`Batch.page_table`, `batch.rs:24-26`,
/// flattened): table `b` is `ids[indptr[b] .. indptr[b + 1]]`.
#[derive(Clone, Debug, Default)]
pub struct Tables {
    pub indptr: Vec<u32>,
    pub ids: Vec<u32>,
}

impl Tables {
    pub fn new() -> Self {
        Self { indptr: vec![0], ids: Vec::new() }
    }
    pub fn push(&mut self, table: &[u32]) {
        self.ids.extend_from_slice(table);
        self.indptr.push(self.ids.len() as u32);
    }
    pub fn len(&self) -> usize {
        self.indptr.len() - 1
    }
    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }
    /// Table `b`.
    pub fn table(&self, b: usize) -> &[u32] {
        &self.ids[self.indptr[b] as usize..self.indptr[b + 1] as usize]
    }
}

/// A decode step's tables split at the leading block ids every table holds
/// (the pages radix sharing handed to every request that matched a prefix,
/// `inference-engine/src/radix_cache.rs:64-117`), limited to blocks that are
/// full before each sequence's last token.
#[derive(Clone, Debug, Default)]
pub struct SharedPrefix {
    /// The shared blocks, in order.
    pub prefix: Vec<u32>,
    /// Each sequence's blocks past the prefix.
    pub suffix_tables: Tables,
    /// Tokens past the prefix (the appended one included), per sequence.
    pub suffix_lens: Vec<i32>,
}

impl SharedPrefix {
    /// `None` when the tables share no leading block.
    pub fn split(tables: &Tables, ctx_lens: &[i32]) -> Option<Self> {
        let b = ctx_lens.len();
        if b == 0 || tables.len() != b {
            return None;
        }
        let mut limit = usize::MAX;
        for (i, &ctx) in ctx_lens.iter().enumerate() {
            let full_before_last = ((ctx.max(1) - 1) as usize) / PAGE_SIZE;
            limit = limit.min(full_before_last).min(tables.table(i).len());
        }
        let first = tables.table(0);
        let n = (0..limit).take_while(|&j| (1..b).all(|i| tables.table(i)[j] == first[j])).count();
        if n == 0 {
            return None;
        }
        let mut suffix_tables = Tables::new();
        for i in 0..b {
            suffix_tables.push(&tables.table(i)[n..]);
        }
        let suffix_lens = ctx_lens.iter().map(|&c| c - (n * PAGE_SIZE) as i32).collect();
        Some(Self { prefix: first[..n].to_vec(), suffix_tables, suffix_lens })
    }
}

/// The device KV pool and the plan of its decode step.
pub struct DeviceKvPool {
    raw: *mut sys::mkv_pool,
    plan: *mut sys::mkv_decode_plan,
    geom: PoolGeometry,
}

// The pool is driven from one thread at a time (the engine's GPU thread);
// the handles are plain heap objects of the library.
unsafe impl Send for DeviceKvPool {}

impl DeviceKvPool {
    /// Allocates the pool on `device` (`MKV_ERR_OUT_OF_MEMORY`, mapped to
    /// `OutOfKvPages`, when HBM cannot hold it) and its decode plan.
    pub fn new(geom: PoolGeometry, device: i32) -> Result<Self, EngineError> {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::mkv_pool_create(&geom.desc(), device, &mut raw) })?;
        let mut plan = ptr::null_mut();
        if let Err(e) = check(unsafe { sys::mkv_decode_plan_create(raw, &mut plan) }) {
            unsafe { sys::mkv_pool_destroy(raw) };
            return Err(e);
        }
        Ok(Self { raw, plan, geom })
    }

    pub fn geometry(&self) -> &PoolGeometry {
        &self.geom
    }

    /// The library handle, for the entry points this type does not wrap
    /// (wire export/import, gathers, device-table forms). The pool keeps
    /// ownership.
    pub fn as_raw(&self) -> *mut sys::mkv_pool {
        self.raw
    }

    /// The pool's device allocation and its size in bytes.
    pub fn buffer(&self) -> Result<(*mut c_void, u64), EngineError> {
        let (mut p, mut n) = (ptr::null_mut(), 0u64);
        check(unsafe { sys::mkv_pool_buffer(self.raw, &mut p, &mut n) })?;
        Ok((p, n))
    }

    /// Once per engine step: the decode requests' host page tables and
    /// context lengths (tokens attended, the one appended this step counted)
    /// into the plan. Validated and copied before the call returns, uploaded
    /// on `stream`; the step's layers then pass no tables.
    pub fn begin_step(&mut self, tables: &Tables, ctx_lens: &[i32], stream: Stream) -> Result<(), EngineError> {
        if tables.len() != ctx_lens.len() {
            return Err(EngineError::Backend(format!(
                "{} page tables for {} context lengths",
                tables.len(),
                ctx_lens.len()
            )));
        }
        check(unsafe {
            sys::mkv_decode_plan_build_tables(
                self.plan,
                ctx_lens.as_ptr(),
                tables.indptr.as_ptr(),
                tables.ids.as_ptr(),
                ctx_lens.len() as i32,
                0,
                stream,
            )
        })
    }

    /// Once per engine step whose decode requests share a prefix: the
    /// plan of `mkv_decode_step_shared_prefix` (the prefix's blocks read once
    /// for every sequence). Validated and copied before the call returns.
    pub fn begin_shared_prefix_step(&mut self, split: &SharedPrefix, stream: Stream) -> Result<(), EngineError> {
        check(unsafe {
            sys::mkv_decode_plan_build_shared_prefix(
                self.plan,
                split.prefix.as_ptr(),
                split.prefix.len() as i32,
                split.suffix_lens.as_ptr(),
                split.suffix_tables.indptr.as_ptr(),
                split.suffix_tables.ids.as_ptr(),
                split.suffix_lens.len() as i32,
                0,
                stream,
            )
        })
    }

    /// One layer of a step planned by `begin_shared_prefix_step`: the same
    /// result as `decode_step` over the whole tables.
    ///
    /// # Safety
    /// As for `decode_step`.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn decode_step_shared_prefix(&mut self, layer: usize, k_new: *const c_void, v_new: *const c_void,
                                            q: *const c_void, o: *mut c_void, scale: f32, flags: u32,
                                            stream: Stream) -> Result<(), EngineError> {
        check(sys::mkv_decode_step_shared_prefix(self.raw, self.plan, layer as i32, k_new, v_new, q, o, ptr::null(),
                                                 0, ptr::null(), ptr::null(), scale, flags, stream))
    }

    /// One layer of the decode step (`inference-model-qwen/src/model.rs:390-416`):
    /// append each request's new K/V row at position `ctx - 1`, then paged
    /// GQA attention over `ctx` tokens, from the plan of `begin_step`.
    ///
    /// # Safety
    /// `k_new`, `v_new` (`[B][Hkv][D]`), `q` and `o` (`[B][Hq][D]`) are device
    /// buffers of the pool's dtype, 16-byte aligned, valid until `stream`
    /// has run the call.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn decode_step(&mut self, layer: usize, k_new: *const c_void, v_new: *const c_void, q: *const c_void,
                              o: *mut c_void, scale: f32, flags: u32, stream: Stream) -> Result<(), EngineError> {
        check(sys::mkv_decode_step(self.raw, self.plan, layer as i32, k_new, v_new, q, o, ptr::null(), ptr::null(),
                                   scale, flags, stream))
    }

    /// K/V rows of prefill tokens into their slots (`slot = table[pos / 16] * 16
    /// + pos % 16`, `prefill.rs:72-81`). The slots are validated and copied
    /// before the call returns.
    ///
    /// # Safety
    /// `k`, `v` are device buffers `[slots.len()][Hkv][D]` of the pool's dtype.
    pub unsafe fn append_host(&mut self, layer: usize, k: *const c_void, v: *const c_void, slots: &[u32],
                              stream: Stream) -> Result<(), EngineError> {
        check(sys::mkv_append_host(self.raw, layer as i32, k, v, slots.as_ptr(), slots.len() as i32, stream))
    }

    /// Causal attention of prefill chunks over their whole caches
    /// (`model.rs:410-416`, mask `:542-555`): request `b`'s `q_lens[b]` query
    /// rows sit at the end of its `ctx_lens[b]` tokens.
    ///
    /// # Safety
    /// `q`, `o` are device buffers `[sum(q_lens)][Hq][D]` of the pool's dtype.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn extend_attention_host(&mut self, layer: usize, q: *const c_void, o: *mut c_void, q_lens: &[i32],
                                        ctx_lens: &[i32], tables: &Tables, scale: f32, flags: u32,
                                        stream: Stream) -> Result<(), EngineError> {
        if q_lens.len() != ctx_lens.len() || tables.len() != ctx_lens.len() {
            return Err(EngineError::Backend("extend attention: lengths and tables differ in count".into()));
        }
        check(sys::mkv_extend_attention_host(self.raw, layer as i32, q, o, q_lens.as_ptr(), ctx_lens.as_ptr(),
                                             tables.indptr.as_ptr(), tables.ids.as_ptr(), q_lens.len() as i32,
                                             scale, flags, stream))
    }

    /// The fused step before attention (`inference-model-qwen/src/model.rs:371-392`):
    /// RMSNorm(1 + w) of every q and k head (`model.rs:104-108`), NeoX RoPE
    /// on their first `rotary_dim` dims at `positions` (`inv_freq` holds
    /// `rotary_dim / 2` frequencies), k and v appended at `slots`; the
    /// prepared q goes to `q_out` `[n][Hq][D]`. `q` is the gated q_proj
    /// output `[n][Hq][2][D]` unless `flags` has `MKV_PREP_PLAIN_Q`. The
    /// positions and slots are validated and copied before the call returns.
    ///
    /// # Safety
    /// `q`, `k`, `v`, `q_out` are device buffers of the pool's dtype; the
    /// weights and frequencies are f32 device buffers (the weights may be
    /// null with `MKV_PREP_NO_NORM`).
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn norm_rope_append_host(&mut self, layer: usize, q: *const c_void, k: *const c_void,
                                        v: *const c_void, q_norm_w: *const f32, k_norm_w: *const f32,
                                        inv_freq: *const f32, rotary_dim: usize, eps: f32, positions: &[i32],
                                        slots: &[u32], q_out: *mut c_void, flags: u32,
                                        stream: Stream) -> Result<(), EngineError> {
        if positions.len() != slots.len() {
            return Err(EngineError::Backend("positions and slots differ in length".into()));
        }
        check(sys::mkv_qk_norm_rope_append_host(self.raw, layer as i32, q, k, v, q_norm_w, k_norm_w, inv_freq,
                                                rotary_dim as i32, eps, positions.as_ptr(), slots.as_ptr(),
                                                slots.len() as i32, q_out, flags, stream))
    }

    /// Copy-on-write copies or compaction moves, every layer, K and V. The
    /// pairs are checked (ids inside the pool, distinct destinations, no
    /// block both a source and a destination) and copied before the call
    /// returns.
    pub fn copy_blocks_host(&mut self, src: &[u32], dst: &[u32], stream: Stream) -> Result<(), EngineError> {
        if src.len() != dst.len() {
            return Err(EngineError::Backend("copy pairs: src and dst differ in length".into()));
        }
        check(unsafe { sys::mkv_copy_blocks_host(self.raw, src.as_ptr(), dst.as_ptr(), src.len() as i32, stream) })
    }

    /// Waits for `stream` and reports an out-of-range id a kernel met (such
    /// an id is skipped, never dereferenced).
    pub fn check(&mut self, stream: Stream) -> Result<(), EngineError> {
        let mut bits = 0u32;
        check(unsafe { sys::mkv_pool_check(self.raw, stream, &mut bits) })
    }

    pub fn synchronize(stream: Stream) -> Result<(), EngineError> {
        check(unsafe { sys::mkv_stream_synchronize(stream) })
    }
}

impl Drop for DeviceKvPool {
    fn drop(&mut self) {
        unsafe {
            sys::mkv_decode_plan_destroy(self.plan);
            sys::mkv_pool_destroy(self.raw);
        }
    }
}
