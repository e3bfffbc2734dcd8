//! The engine's page lifecycle on the host block manager (`libmitten_kvhost`).
//!
//! The reference keeps an allocator (`inference-engine/src/kv_pool.rs`) and a
//! radix tree (`radix_cache.rs`) side by side with no per-page reference
//! counts: pages matched from the tree are freed again on Done
//! (`scheduler.rs:169-171`), decode never grows a table (`scheduler.rs:133`)
//! and shared pages are aliased, never copied. The block manager replaces
//! both with reference-counted blocks, decode-time growth, copy-on-write and
//! compaction; [`PagedLifecycle`] makes its calls at the reference's sites
//! and queues the block copies they imply for the backend, which runs them
//! on its stream before the next step reads the pool.

use crate::error::check_host;
use inference_backend::{EngineError, KvPool, Request, RequestId, RequestState};
use mitten_kvhost_sys as hsys;
use parking_lot::Mutex;
use std::collections::{HashMap, VecDeque};
use std::ptr;
use std::sync::Arc;

/// The chunking rule of `PrefillAdder` (`prefill.rs:27-36,99-114`) over
/// in-progress prefills, in order: each gets `min(remaining, budget - used)`
/// tokens until the budget is used up. Returns (chunks, tokens used).
pub fn schedule_prefill_chunks(budget: usize, remaining: &[usize]) -> Result<(Vec<usize>, usize), EngineError> {
    let rem: Vec<i64> = remaining.iter().map(|&r| r as i64).collect();
    let mut out = vec![0i64; rem.len()];
    let mut used = 0i64;
    check_host(unsafe {
        hsys::mkvh_schedule_prefill_chunks(budget as i64, rem.as_ptr(), rem.len() as i32, out.as_mut_ptr(), &mut used)
    })?;
    Ok((out.into_iter().map(|c| c as usize).collect(), used as usize))
}

/// Slots of an append and the copy-on-write pair that must run before it.
#[derive(Clone, Debug, Default)]
pub struct Appended {
    pub slots: Vec<u32>,
    pub cow: Option<(u32, u32)>,
}

/// One step's prefill schedule (`PrefillAdder::run`, `prefill.rs:21-114`).
#[derive(Clone, Debug, Default)]
pub struct PrefillSchedule {
    /// Chunk of each in-progress prefill, in the order given (0: none).
    pub in_progress: Vec<usize>,
    /// Chunk of each admitted waiting request (0: its whole prompt was cached).
    pub admitted: Vec<usize>,
    /// Radix hits of the admitted requests.
    pub cached_lens: Vec<usize>,
}

/// Reference-counted blocks of the engine's sequences over the device pool.
pub struct HostBlockManager {
    raw: *mut hsys::mkvh_block_manager,
    num_blocks: usize,
}

unsafe impl Send for HostBlockManager {}

impl HostBlockManager {
    /// `num_blocks` blocks of 16 tokens; the radix tree may cache up to
    /// `max_cached_pages` of them (`radix_cache.rs:37-62`).
    pub fn new(num_blocks: usize, max_cached_pages: usize) -> Result<Self, EngineError> {
        let mut raw = ptr::null_mut();
        check_host(unsafe {
            hsys::mkvh_bm_create(num_blocks as i64, crate::PAGE_SIZE as i32, max_cached_pages as i64, &mut raw)
        })?;
        Ok(Self { raw, num_blocks })
    }

    pub fn num_blocks(&self) -> usize {
        self.num_blocks
    }

    /// Admission (`prefill.rs:39-81`): evict the deficit once, match the
    /// prompt's full pages in the tree (shared, locked), allocate the rest.
    /// Returns the cached length; `OutOfKvPages` (and no change) when the
    /// pool cannot hold the prompt.
    pub fn admit(&mut self, seq: u64, prompt: &[u32]) -> Result<usize, EngineError> {
        let mut cached = 0i64;
        check_host(unsafe { hsys::mkvh_bm_admit(self.raw, seq, prompt.as_ptr(), prompt.len() as i64, &mut cached) })?;
        Ok(cached as usize)
    }

    /// A new sequence sharing every block of `parent` (parallel sampling).
    pub fn fork(&mut self, parent: u64, child: u64) -> Result<(), EngineError> {
        check_host(unsafe { hsys::mkvh_bm_fork(self.raw, parent, child) })
    }

    /// Slots of `n_new` tokens at the sequence's end; a block is allocated
    /// where a position starts one, and a shared block is made private first.
    pub fn append(&mut self, seq: u64, n_new: usize) -> Result<Appended, EngineError> {
        let mut slots = vec![0i32; n_new.max(1)];
        let (mut src, mut dst, mut n_cow) = (0i32, 0i32, 0i32);
        check_host(unsafe {
            hsys::mkvh_bm_append(self.raw, seq, n_new as i32, slots.as_mut_ptr(), &mut src, &mut dst, &mut n_cow)
        })?;
        slots.truncate(n_new);
        Ok(Appended {
            slots: slots.into_iter().map(|s| s as u32).collect(),
            cow: if n_cow > 0 { Some((src as u32, dst as u32)) } else { None },
        })
    }

    /// `PrefillAdder::run` on these books: in-progress prefills first, then
    /// waiting prompts admitted in order while budget remains.
    pub fn schedule_prefill(&mut self, budget: usize, in_progress: &[u64],
                            waiting: &[(u64, &[u32])]) -> Result<PrefillSchedule, EngineError> {
        let wseq: Vec<u64> = waiting.iter().map(|w| w.0).collect();
        let mut indptr = Vec::with_capacity(waiting.len() + 1);
        let mut tokens: Vec<u32> = Vec::new();
        indptr.push(0i64);
        for (_, t) in waiting {
            tokens.extend_from_slice(t);
            indptr.push(tokens.len() as i64);
        }
        let mut chunks = vec![0i64; in_progress.len() + waiting.len()];
        let mut cached = vec![0i64; waiting.len()];
        let mut n_admitted = 0i32;
        check_host(unsafe {
            hsys::mkvh_bm_schedule_prefill(self.raw, budget as i64, in_progress.as_ptr(), in_progress.len() as i32,
                                           wseq.as_ptr(), indptr.as_ptr(), tokens.as_ptr(), wseq.len() as i32,
                                           chunks.as_mut_ptr(), &mut n_admitted, cached.as_mut_ptr())
        })?;
        let k = n_admitted as usize;
        let ip = in_progress.len();
        Ok(PrefillSchedule {
            in_progress: chunks[..ip].iter().map(|&c| c as usize).collect(),
            admitted: chunks[ip..ip + k].iter().map(|&c| c as usize).collect(),
            cached_lens: cached[..k].iter().map(|&c| c as usize).collect(),
        })
    }

    /// Prefill complete (`scheduler.rs:117`): full pages enter the tree.
    pub fn promote(&mut self, seq: u64, tokens: &[u32]) -> Result<(), EngineError> {
        check_host(unsafe { hsys::mkvh_bm_promote(self.raw, seq, tokens.as_ptr(), tokens.len() as i64) })
    }

    /// Done / Aborted (`scheduler.rs:164-172`, `decode.rs:20-33`).
    pub fn release(&mut self, seq: u64) -> Result<(), EngineError> {
        check_host(unsafe { hsys::mkvh_bm_release(self.raw, seq) })
    }

    /// LRU eviction of tree leaves; returns the blocks freed.
    pub fn evict(&mut self, target_pages: usize) -> Result<usize, EngineError> {
        let mut freed = 0i64;
        check_host(unsafe { hsys::mkvh_bm_evict(self.raw, target_pages as i64, &mut freed) })?;
        Ok(freed as usize)
    }

    /// Block moves that pack the live blocks below the live count; the
    /// sequences' tables and the tree's pages are rewritten.
    pub fn plan_compaction(&mut self) -> Result<(Vec<u32>, Vec<u32>), EngineError> {
        let cap = self.num_blocks.max(1);
        let (mut src, mut dst) = (vec![0i32; cap], vec![0i32; cap]);
        let mut n = 0i64;
        check_host(unsafe {
            hsys::mkvh_bm_plan_compaction(self.raw, src.as_mut_ptr(), dst.as_mut_ptr(), cap as i64, &mut n)
        })?;
        let n = n as usize;
        Ok((src[..n].iter().map(|&b| b as u32).collect(), dst[..n].iter().map(|&b| b as u32).collect()))
    }

    /// The sequence's block table (its `kv_pages`, `request.rs:53-54`).
    pub fn table(&self, seq: u64) -> Result<Vec<u32>, EngineError> {
        let cap = self.num_blocks.max(1) as i64;
        let mut out = vec![0i32; cap as usize];
        let mut n = 0i64;
        check_host(unsafe { hsys::mkvh_bm_table(self.raw, seq, out.as_mut_ptr(), cap, &mut n) })?;
        Ok(out[..n as usize].iter().map(|&b| b as u32).collect())
    }

    pub fn seq_len(&self, seq: u64) -> Result<usize, EngineError> {
        let mut len = 0i64;
        check_host(unsafe { hsys::mkvh_bm_seq_len(self.raw, seq, &mut len) })?;
        Ok(len as usize)
    }

    pub fn free_blocks(&self) -> usize {
        unsafe { hsys::mkvh_bm_free_blocks(self.raw) as usize }
    }

    pub fn live_blocks(&self) -> usize {
        unsafe { hsys::mkvh_bm_live_blocks(self.raw) as usize }
    }

    /// Every live block's count equals its holders; free + live = total.
    pub fn check_invariants(&self) -> Result<(), EngineError> {
        check_host(unsafe { hsys::mkvh_bm_check_invariants(self.raw) })
    }
}

impl Drop for HostBlockManager {
    fn drop(&mut self) {
        unsafe { hsys::mkvh_bm_destroy(self.raw) }
    }
}

/// Block copies planned on the scheduler thread, run by the backend on its
/// stream before the next step: groups in order, each group one
/// `mkv_copy_blocks_host` call (its pairs are independent of each other).
pub type CopyQueue = Arc<Mutex<VecDeque<(Vec<u32>, Vec<u32>)>>>;

/// `BackendHandle::kv_pool()` (`backend.rs:19,23-26`): the block manager's
/// counts.
pub struct PoolView {
    bm: Arc<Mutex<HostBlockManager>>,
}

impl KvPool for PoolView {
    fn free_pages(&self) -> usize {
        self.bm.lock().free_blocks()
    }
    fn total_pages(&self) -> usize {
        self.bm.lock().num_blocks()
    }
}

/// The scheduler's side of the paged pool. Each method names the reference
/// site it replaces.
pub struct PagedLifecycle {
    bm: Arc<Mutex<HostBlockManager>>,
    copies: CopyQueue,
    seqs: HashMap<RequestId, u64>,
    next_seq: u64,
}

impl PagedLifecycle {
    pub fn new(num_blocks: usize, max_cached_pages: usize) -> Result<Self, EngineError> {
        Ok(Self {
            bm: Arc::new(Mutex::new(HostBlockManager::new(num_blocks, max_cached_pages)?)),
            copies: Arc::new(Mutex::new(VecDeque::new())),
            seqs: HashMap::new(),
            next_seq: 1,
        })
    }

    /// Blocks of the pool the books describe.
    pub fn num_blocks(&self) -> usize {
        self.bm.lock().num_blocks()
    }

    /// The view the backend returns from `kv_pool()`.
    pub fn pool_view(&self) -> PoolView {
        PoolView { bm: self.bm.clone() }
    }

    /// The queue the backend drains at the start of each forward.
    pub fn copy_queue(&self) -> CopyQueue {
        self.copies.clone()
    }

    fn seq_of(&mut self, id: RequestId) -> u64 {
        let next = &mut self.next_seq;
        *self.seqs.entry(id).or_insert_with(|| {
            let s = *next;
            *next += 1;
            s
        })
    }

    fn known(&self, id: RequestId) -> Result<u64, EngineError> {
        self.seqs.get(&id).copied().ok_or_else(|| EngineError::Backend(format!("request {id} holds no blocks")))
    }

    /// `PrefillAdder::run` (`prefill.rs:21-114`) with `budget` =
    /// `max_prefill_tokens_per_iter - decode tokens` (`scheduler.rs:14-18`).
    /// In-progress prefills first, then admission from the front of
    /// `waiting` while budget remains. Admitted requests leave `waiting` with
    /// their `cached_len`, `device_len`, `kv_pages` and `Prefilling` state set
    /// and are returned second (the engine appends them to its prefilling
    /// list); the requests to run this step, with `extend_len` set, first.
    pub fn schedule_prefill(&mut self, budget: usize, prefilling: &[Arc<Mutex<Request>>],
                            waiting: &mut VecDeque<Arc<Mutex<Request>>>)
                            -> Result<(Vec<Arc<Mutex<Request>>>, Vec<Arc<Mutex<Request>>>), EngineError> {
        let ip: Vec<u64> = prefilling.iter().map(|r| self.known(r.lock().id)).collect::<Result<_, _>>()?;
        let cand: Vec<Arc<Mutex<Request>>> = waiting.iter().cloned().collect();
        let prompts: Vec<Vec<u32>> = cand.iter().map(|r| r.lock().input_ids.clone()).collect();
        let ids: Vec<u64> = cand.iter().map(|r| { let id = r.lock().id; self.seq_of(id) }).collect();
        let wait: Vec<(u64, &[u32])> = ids.iter().copied().zip(prompts.iter().map(|p| p.as_slice())).collect();
        let sched = self.bm.lock().schedule_prefill(budget, &ip, &wait)?;
        // Requests not admitted keep no sequence id.
        for r in &cand[sched.admitted.len()..] {
            self.seqs.remove(&r.lock().id);
        }
        let mut run = Vec::new();
        for (r, &chunk) in prefilling.iter().zip(&sched.in_progress) {
            if chunk > 0 {
                r.lock().extend_len = chunk;
                run.push(r.clone());
            }
        }
        let mut admitted = Vec::new();
        for (i, &chunk) in sched.admitted.iter().enumerate() {
            let r = waiting.pop_front().expect("admitted requests are the front of the waiting queue");
            {
                let mut req = r.lock();
                req.cached_len = sched.cached_lens[i];
                req.device_len = sched.cached_lens[i];
                req.kv_pages = self.bm.lock().table(ids[i])?;
                req.state = RequestState::Prefilling { processed_tokens: 0 };
                req.extend_len = chunk;
            }
            if chunk > 0 {
                run.push(r.clone());
            }
            admitted.push(r);
        }
        Ok((run, admitted))
    }

    /// Before the step's batch is assembled (`scheduler.rs:29-77`): the
    /// tokens each request writes this step (`extend_len` for prefills, one
    /// for decodes) get their slots; a table grows where a position starts a
    /// block, and a shared block about to be written is made private, its
    /// copy queued for the backend. `kv_pages` is refreshed, so the batch's
    /// page tables cover the step.
    pub fn prepare_step(&mut self, prefill: &[Arc<Mutex<Request>>], decode: &[Arc<Mutex<Request>>])
                        -> Result<(), EngineError> {
        let (mut src, mut dst) = (Vec::new(), Vec::new());
        for (reqs, is_prefill) in [(prefill, true), (decode, false)] {
            for r in reqs {
                let mut req = r.lock();
                let seq = self.known(req.id)?;
                let n = if is_prefill { req.extend_len } else { 1 };
                let mut bm = self.bm.lock();
                let app = bm.append(seq, n)?;
                if let Some((s, d)) = app.cow {
                    src.push(s);
                    dst.push(d);
                }
                req.kv_pages = bm.table(seq)?;
            }
        }
        if !src.is_empty() {
            self.copies.lock().push_back((src, dst));
        }
        Ok(())
    }

    /// Prefill complete (`scheduler.rs:117`, `radix_cache.rs:287-294`).
    pub fn promote(&mut self, req: &Request) -> Result<(), EngineError> {
        let seq = self.known(req.id)?;
        self.bm.lock().promote(seq, &req.input_ids)
    }

    /// Done or Aborted (`scheduler.rs:164-172`, `decode.rs:20-33`): the
    /// request's references go; pages the tree holds survive (the
    /// reference frees them a second time, `kv_pool.rs:41-44`).
    pub fn release(&mut self, req: &mut Request) -> Result<(), EngineError> {
        let seq = self.known(req.id)?;
        self.bm.lock().release(seq)?;
        self.seqs.remove(&req.id);
        req.kv_pages.clear();
        req.locked_nodes.clear();
        Ok(())
    }

    /// LRU eviction of `target_pages` tree pages (`radix_cache.rs:243-282`),
    /// then compaction: the moves are queued for the backend and every live
    /// request's `kv_pages` is rewritten. Returns the blocks freed.
    pub fn evict_and_compact(&mut self, target_pages: usize, live: &[Arc<Mutex<Request>>])
                             -> Result<usize, EngineError> {
        let mut bm = self.bm.lock();
        let freed = bm.evict(target_pages)?;
        let (src, dst) = bm.plan_compaction()?;
        if !src.is_empty() {
            self.copies.lock().push_back((src, dst));
        }
        for r in live {
            let mut req = r.lock();
            if let Some(&seq) = self.seqs.get(&req.id) {
                req.kv_pages = bm.table(seq)?;
            }
        }
        Ok(freed)
    }
}
