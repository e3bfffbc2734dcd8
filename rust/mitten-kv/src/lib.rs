//! Paged KV cache for the mitten engine on one AMD MI355X.
//!
//! The reference backend keeps a private contiguous cache per request and
//! drops the scheduler's page tables (`inference-backend/src/burn_backend.rs:44-71`).
//! This crate puts a device KV pool behind the engine's own page tables:
//!
//! * [`DeviceKvPool`]: the backend's device-buffer type. One HBM allocation
//!   laid out `[layer][K|V][block][16 tokens][kv head][head dim]`, sized as
//!   `KvCachePool::required_bytes` (`inference-engine/src/kv_pool.rs:58-68`),
//!   with the decode step's plan. Every operation is a `libmitten_kv` call.
//! * [`HostBlockManager`]: the engine's page bookkeeping with per-block
//!   reference counts, decode-time growth, copy-on-write, compaction and the
//!   prefill budget rule (`libmitten_kvhost`).
//! * [`PagedLifecycle`]: the scheduler-side calls at the reference's
//!   admission, promotion, release and eviction sites
//!   (`prefill.rs:21-114`, `scheduler.rs:117`, `scheduler.rs:164-172`,
//!   `decode.rs:20-33`); block copies it plans are queued for the backend.
//! * [`PagedBackend`]: an `inference_backend::BackendHandle`
//!   (`inference-backend/src/backend.rs:16-26`) whose `forward` runs the
//!   queued block copies, builds the step's plan once from the batch's page
//!   tables, and per layer appends and attends through the pool; the model
//!   crates supply everything else through [`PagedModel`].

mod backend;
mod error;
mod host;
mod pool;

pub use backend::{AttentionIo, PagedBackend, PagedModel, StepLayout, SHARED_PREFIX_MIN_BYTES};
pub use error::check;
pub use host::{
    schedule_prefill_chunks, Appended, CopyQueue, HostBlockManager, PagedLifecycle, PoolView, PrefillSchedule,
};
pub use pool::{DeviceKvPool, KvDtype, PoolGeometry, SharedPrefix, Stream, Tables, PAGE_SIZE};
