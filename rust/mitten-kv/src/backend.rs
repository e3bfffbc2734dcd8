//! `PagedBackend`: the engine's `BackendHandle` (`inference-backend/src/backend.rs:16-26`)
//! over the device KV pool.
//!
//! The reference's `BurnBackend::forward` (`burn_backend.rs:31-80`) runs each
//! request alone over a private cache grown by `Tensor::cat`
//! (`inference-model-qwen/src/model.rs:390-392`). Here one forward covers the
//! whole batch: prefill chunks first, then decode tokens, in the order
//! `assemble_batch` builds (`inference-engine/src/scheduler.rs:29-77`), and
//! per attention layer the pool is the KV cache:
//!
//! * prefill rows: their K/V into their slots (`mkv_append_host`), then causal
//!   attention over each request's whole cache (`mkv_extend_attention_host`);
//! * decode rows: one `mkv_decode_step` (append + paged attention) from the
//!   plan `begin_step` built once for the step.
//!
//! Everything else in a layer (projections, q/k norm, RoPE, gate, o_proj,
//! MLP) belongs to the model; the model crates expose it through [`PagedModel`].

use crate::host::{CopyQueue, PagedLifecycle, PoolView};
use crate::pool::{DeviceKvPool, KvDtype, PoolGeometry, SharedPrefix, Stream, Tables, PAGE_SIZE};
// BoxFuture is not re-exported at the crate root (inference-backend/src/lib.rs:10).
use inference_backend::backend::BoxFuture;
use inference_backend::{BackendHandle, Batch, EngineError, KvPool, Logits, ModelConfig, RequestState};
use mitten_kv_sys as sys;
use parking_lot::Mutex;
use std::ffi::c_void;

/// Device buffers of one layer's attention for every row of the batch, in
/// batch order: q and o `[rows][Hq][D]`, k and v `[rows][Hkv][D]`, the pool's
/// dtype, 16-byte aligned. q and k carry the layer's norm and RoPE.
#[derive(Clone, Copy, Debug)]
pub struct AttentionIo {
    pub q: *const c_void,
    pub k: *const c_void,
    pub v: *const c_void,
    pub o: *mut c_void,
}

/// The model side of a paged forward: a layer stack split at the attention
/// call (`inference-model-qwen/src/model.rs:390-416`; Gemma's attention at
/// `inference-model-gemma/src/model.rs`). All work is enqueued on `stream`.
pub trait PagedModel: Send {
    /// Query heads of the attention layers (absent from `ModelConfig`).
    fn num_q_heads(&self) -> usize;
    /// Embeds the batch's tokens (`Batch.input_ids`, positions
    /// `Batch.position_ids`) as the first layer's input.
    fn begin(&mut self, input_ids: &[u32], position_ids: &[u32], stream: Stream) -> Result<(), EngineError>;
    /// Runs layer `layer` up to its attention and returns the attention's
    /// buffers (`model.rs:369-384`).
    fn attention_io(&mut self, layer: usize, stream: Stream) -> Result<AttentionIo, EngineError>;
    /// Consumes the attention output in `o` and finishes the layer
    /// (`model.rs:417-418` and the MLP).
    fn finish_layer(&mut self, layer: usize, stream: Stream) -> Result<(), EngineError>;
    /// Logits of the given rows, one `vocab_size` row each, in order.
    fn logits(&mut self, rows: &[usize], stream: Stream) -> Result<Vec<f32>, EngineError>;
}

/// The step's metadata from the batch: prefill requests (chunks) then
/// decode requests, their slots, lengths and page tables.
#[derive(Clone, Debug, Default)]
pub struct StepLayout {
    /// Rows (tokens) of the prefill chunks; decode rows follow them.
    pub prefill_rows: usize,
    pub prefill_slots: Vec<u32>,
    pub prefill_q_lens: Vec<i32>,
    pub prefill_ctx: Vec<i32>,
    pub prefill_tables: Tables,
    pub decode_ctx: Vec<i32>,
    pub decode_tables: Tables,
    /// One row per request: a prefill chunk's last token, or the decode token.
    pub logit_rows: Vec<usize>,
}

fn slot(table: &[u32], pos: usize, what: &dyn std::fmt::Display) -> Result<u32, EngineError> {
    match table.get(pos / PAGE_SIZE) {
        Some(&page) => Ok(page * PAGE_SIZE as u32 + (pos % PAGE_SIZE) as u32),
        None => Err(EngineError::Backend(format!(
            "request {what}: position {pos} lies past its {} pages",
            table.len()
        ))),
    }
}

impl StepLayout {
    /// Reads the batch as `assemble_batch` builds it: a prefill request
    /// writes `extend_len` tokens at positions `device_len..` and attends over
    /// `device_len + extend_len` of them; a decode request writes one token at
    /// `device_len` and attends over `device_len + 1` (`scheduler.rs:39-57`).
    pub fn new(batch: &Batch) -> Result<Self, EngineError> {
        if batch.page_table.len() != batch.requests.len() {
            return Err(EngineError::Backend("one page table per request expected".into()));
        }
        let mut s = StepLayout { prefill_tables: Tables::new(), decode_tables: Tables::new(), ..Default::default() };
        let mut rows = 0usize;
        for (req_arc, table) in batch.requests.iter().zip(&batch.page_table) {
            let req = req_arc.lock();
            match req.state {
                RequestState::Prefilling { .. } => {
                    if !s.decode_ctx.is_empty() {
                        return Err(EngineError::Backend("a prefill request follows a decode request".into()));
                    }
                    let (start, n) = (req.device_len, req.extend_len);
                    if n == 0 {
                        return Err(EngineError::Backend(format!("prefill request {} has no chunk", req.id)));
                    }
                    for pos in start..start + n {
                        s.prefill_slots.push(slot(table, pos, &req.id)?);
                    }
                    s.prefill_q_lens.push(n as i32);
                    s.prefill_ctx.push((start + n) as i32);
                    s.prefill_tables.push(table);
                    rows += n;
                }
                RequestState::Decoding => {
                    slot(table, req.device_len, &req.id)?;
                    s.decode_ctx.push((req.device_len + 1) as i32);
                    s.decode_tables.push(table);
                    rows += 1;
                }
                _ => {
                    return Err(EngineError::Backend(format!("request {} is neither prefilling nor decoding", req.id)))
                }
            }
            s.logit_rows.push(rows - 1);
        }
        s.prefill_rows = rows - s.decode_ctx.len();
        if rows != batch.input_ids.len() {
            return Err(EngineError::Backend(format!(
                "the batch has {} input ids for {rows} rows",
                batch.input_ids.len()
            )));
        }
        Ok(s)
    }
}

/// A `Send` wrapper of the backend's stream handle.
#[derive(Clone, Copy)]
struct StreamHandle(Stream);
unsafe impl Send for StreamHandle {}

struct Inner<M> {
    pool: DeviceKvPool,
    model: M,
    stream: StreamHandle,
}

/// The paged backend. `forward` runs on the engine's GPU thread
/// (`inference-api/src/main.rs:84-91`); the lock only makes `&self` calls
/// exclusive, it is never contended there.
pub struct PagedBackend<M: PagedModel> {
    inner: Mutex<Inner<M>>,
    config: ModelConfig,
    view: PoolView,
    copies: CopyQueue,
    scale: f32,
    flags: u32,
    shared_prefix_min_bytes: u64,
}

/// K/V bytes per layer a shared prefix must save (its blocks read once
/// instead of once per sequence) before a step takes the shared-prefix form,
/// whose prefix tiles and merge cost about two extra launches per layer.
pub const SHARED_PREFIX_MIN_BYTES: u64 = 128 << 20;

impl<M: PagedModel> PagedBackend<M> {
    /// A pool on `device` for `model` with as many blocks as the scheduler's
    /// block manager (`lifecycle`) hands out, sharing its books. `zero_sink`
    /// reproduces the Qwen reference's phantom zero slot (`model.rs:207-220`)
    /// exactly.
    pub fn new(model: M, config: ModelConfig, lifecycle: &PagedLifecycle, dtype: KvDtype, device: i32,
               stream: Stream, zero_sink: bool) -> Result<Self, EngineError> {
        let geom = PoolGeometry::from_model(&config, model.num_q_heads(), lifecycle.num_blocks(), dtype);
        let pool = DeviceKvPool::new(geom, device)?;
        Ok(Self {
            inner: Mutex::new(Inner { pool, model, stream: StreamHandle(stream) }),
            scale: (config.head_dim as f32).powf(-0.5),
            flags: if zero_sink { sys::MKV_ATTN_ZERO_SINK } else { 0 },
            config,
            view: lifecycle.pool_view(),
            copies: lifecycle.copy_queue(),
            shared_prefix_min_bytes: SHARED_PREFIX_MIN_BYTES,
        })
    }

    /// Bytes per layer a shared prefix must save before a step reads it
    /// once for all its decode requests (`u64::MAX`: never).
    pub fn with_shared_prefix_min_bytes(mut self, bytes: u64) -> Self {
        self.shared_prefix_min_bytes = bytes;
        self
    }

    /// The step's decode tables split at a prefix every request shares, when
    /// the geometry takes the shared-prefix step and the prefix saves enough.
    fn shared_prefix(&self, geom: &PoolGeometry, step: &StepLayout) -> Option<SharedPrefix> {
        let b = step.decode_ctx.len();
        if b < 2 || !geom.shared_prefix_supported() {
            return None;
        }
        let split = SharedPrefix::split(&step.decode_tables, &step.decode_ctx)?;
        let block_bytes = (2 * PAGE_SIZE * geom.kv_row_bytes()) as u64;
        let saved = (b as u64 - 1) * split.prefix.len() as u64 * block_bytes;
        (saved >= self.shared_prefix_min_bytes).then_some(split)
    }

    fn forward_now(&self, batch: &Batch) -> Result<Logits, EngineError> {
        let step = StepLayout::new(batch)?;
        let mut guard = self.inner.lock();
        let inner = &mut *guard;
        let stream = inner.stream.0;
        // Block copies the scheduler planned (copy-on-write before this
        // step's appends, compaction moves), in order, before any read.
        loop {
            let group = self.copies.lock().pop_front();
            match group {
                Some((src, dst)) => inner.pool.copy_blocks_host(&src, &dst, stream)?,
                None => break,
            }
        }
        let geom = *inner.pool.geometry();
        // Decode requests that share a radix prefix read its blocks once for
        // all of them (mkv_decode_step_shared_prefix); otherwise one plan of
        // their whole tables.
        let shared = self.shared_prefix(&geom, &step);
        match &shared {
            Some(split) => inner.pool.begin_shared_prefix_step(split, stream)?,
            None if !step.decode_ctx.is_empty() => {
                inner.pool.begin_step(&step.decode_tables, &step.decode_ctx, stream)?
            }
            None => {}
        }
        inner.model.begin(&batch.input_ids, &batch.position_ids, stream)?;
        let (kv_off, q_off) = (step.prefill_rows * geom.kv_row_bytes(), step.prefill_rows * geom.q_row_bytes());
        for layer in 0..geom.num_layers {
            let io = inner.model.attention_io(layer, stream)?;
            // SAFETY: the model's buffers hold every row of the batch
            // (AttentionIo), so the decode rows start `prefill_rows` rows in.
            unsafe {
                if step.prefill_rows > 0 {
                    inner.pool.append_host(layer, io.k, io.v, &step.prefill_slots, stream)?;
                    inner.pool.extend_attention_host(layer, io.q, io.o, &step.prefill_q_lens, &step.prefill_ctx,
                                                     &step.prefill_tables, self.scale, self.flags, stream)?;
                }
                if !step.decode_ctx.is_empty() {
                    let at = |p: *const c_void, off: usize| p.cast::<u8>().wrapping_add(off).cast::<c_void>();
                    let o = io.o.cast::<u8>().wrapping_add(q_off).cast::<c_void>();
                    let (k, v, q) = (at(io.k, kv_off), at(io.v, kv_off), at(io.q, q_off));
                    if shared.is_some() {
                        inner.pool.decode_step_shared_prefix(layer, k, v, q, o, self.scale, self.flags, stream)?;
                    } else {
                        inner.pool.decode_step(layer, k, v, q, o, self.scale, self.flags, stream)?;
                    }
                }
            }
            inner.model.finish_layer(layer, stream)?;
        }
        let data = inner.model.logits(&step.logit_rows, stream)?;
        inner.pool.check(stream)?;
        Ok(Logits { data, num_rows: batch.requests.len(), vocab_size: self.config.vocab_size })
    }
}

impl<M: PagedModel + 'static> BackendHandle for PagedBackend<M> {
    fn forward(&self, batch: &Batch) -> BoxFuture<'_, Result<Logits, EngineError>> {
        let out = self.forward_now(batch);
        Box::pin(async move { out })
    }

    fn kv_pool(&self) -> &dyn KvPool {
        &self.view
    }

    fn model_config(&self) -> &ModelConfig {
        &self.config
    }
}
