"""Seeded synthetic decode batches at the shapes of the benchmark configurations.

Integers come from SplitMix64 with Lemire's bounded draw, so every length,
permutation and slot below is a pure function of the seed. A decode batch is
what one engine step hands the device: per sequence a block table (CSR), the
number of tokens to attend (context + the token appended this step) and the
slot of the appended token, slot = table[pos // 16] * 16 + pos % 16
(inference-engine/src/prefill.rs:72-81, scheduler.rs:56-57).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

PAGE = 16
MASK64 = (1 << 64) - 1
BASE_SEED = 20261201


class SplitMix64:
    def __init__(self, seed: int):
        self.s = seed & MASK64

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & MASK64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        return z ^ (z >> 31)

    def bounded(self, n: int) -> int:
        """Uniform in [0, n), Lemire's multiply-shift with rejection."""
        x = self.next() >> 32
        m = x * n
        lo = m & 0xFFFFFFFF
        if lo < n:
            t = (-n & 0xFFFFFFFF) % n
            while lo < t:
                x = self.next() >> 32
                m = x * n
                lo = m & 0xFFFFFFFF
        return m >> 32

    def uniform_int(self, lo: int, hi: int) -> int:
        return lo + self.bounded(hi - lo + 1)

    def uniform01(self) -> float:
        return ((self.next() >> 11) + 1) * (1.0 / 9007199254740992.0)


def permutation(n: int, rng: SplitMix64) -> np.ndarray:
    """Fisher-Yates shuffle of 0..n-1."""
    p = np.arange(n, dtype=np.int32)
    for i in range(n - 1, 0, -1):
        j = rng.bounded(i + 1)
        p[i], p[j] = p[j], p[i]
    return p


@dataclass
class DecodeBatch:
    ctx_lens: np.ndarray       # int32 [B]: tokens attended (existing context + 1)
    block_indptr: np.ndarray   # int32 [B+1]
    block_ids: np.ndarray      # int32 [nnz]
    slot_mapping: np.ndarray   # int32 [B]: slot of the appended token
    num_blocks: int            # pool blocks covering every table
    seed: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return int(self.ctx_lens.size)

    @property
    def max_ctx(self) -> int:
        return int(self.ctx_lens.max())

    @property
    def total_tokens(self) -> int:
        return int(self.ctx_lens.sum())

    @property
    def ctx_indptr(self) -> np.ndarray:
        out = np.zeros(self.num_seqs + 1, np.int32)
        np.cumsum(self.ctx_lens, out=out[1:])
        return out


def decode_batch_from_contexts(contexts, rng: SplitMix64, extra_blocks: int = 0,
                               shuffle: bool = True) -> DecodeBatch:
    """Each sequence holds `contexts[b]` tokens and appends one at position
    contexts[b]; its table covers ceil((ctx+1)/16) blocks. Tables are slices of
    a seeded permutation of the pool ids (or of 0..n-1 when shuffle=False)."""
    ctx = np.asarray(contexts, np.int64)
    attend = ctx + 1
    nblk = (attend + PAGE - 1) // PAGE
    total = int(nblk.sum())
    num_blocks = total + extra_blocks
    perm = permutation(num_blocks, rng) if shuffle else np.arange(num_blocks, dtype=np.int32)
    indptr = np.zeros(ctx.size + 1, np.int32)
    np.cumsum(nblk, out=indptr[1:])
    ids = perm[:total].astype(np.int32)
    pos = ctx
    slots = ids[indptr[:-1] + pos // PAGE].astype(np.int64) * PAGE + pos % PAGE
    return DecodeBatch(attend.astype(np.int32), indptr, ids, slots.astype(np.int32), num_blocks)


def uniform_contexts(B: int, lo: int, hi: int, rng: SplitMix64):
    return [rng.uniform_int(lo, hi) for _ in range(B)]


def lognormal_lengths(rng: SplitMix64, n: int, median: int, sigma: float, cap: int) -> list[int]:
    """n lengths median * exp(sigma * z), z ~ N(0,1) by Box-Muller, rounded
    and clamped to [1, cap]."""
    out = []
    for _ in range(n):
        u1, u2 = rng.uniform01(), rng.uniform01()
        z = math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)
        out.append(int(min(cap, max(1, round(median * math.exp(sigma * z))))))
    return out


def shared_prefix_batch(num_seqs: int, prefix: int, suffix_lo: int, suffix_hi: int,
                        rng: SplitMix64) -> DecodeBatch:
    """A decode step after radix sharing and copy-on-write: every sequence
    holds `prefix` shared tokens plus a suffix ~U{suffix_lo..suffix_hi} and
    appends one token. Its table starts with the prefix's full blocks, the
    same ids in every table (refcounted, read by every sequence), followed by
    its own blocks: its copy of the prefix's partial block and its suffix.
    Ids come from a seeded permutation of the pool. meta["shared_blocks"]
    holds the shared ids, meta["own_first"] each sequence's first own block
    (its copy of the partial block) and meta["unique_tokens"] the tokens
    attended once each: the shared blocks' tokens once plus every
    sequence's own tokens."""
    full = prefix // PAGE
    ctx = np.asarray([prefix + rng.uniform_int(suffix_lo, suffix_hi) for _ in range(num_seqs)], np.int64)
    attend = ctx + 1
    own = (attend + PAGE - 1) // PAGE - full
    num_blocks = full + int(own.sum())
    perm = permutation(num_blocks, rng)
    shared = perm[:full]
    indptr = np.zeros(num_seqs + 1, np.int32)
    np.cumsum(own + full, out=indptr[1:])
    ids = np.empty(int(indptr[-1]), np.int32)
    nxt = full
    own_first = np.empty(num_seqs, np.int32)
    for b in range(num_seqs):
        o = int(own[b])
        ids[indptr[b]:indptr[b] + full] = shared
        ids[indptr[b] + full:indptr[b + 1]] = perm[nxt:nxt + o]
        own_first[b] = perm[nxt]
        nxt += o
    slots = ids[indptr[:-1] + ctx // PAGE].astype(np.int64) * PAGE + ctx % PAGE
    unique = full * PAGE + int((attend - full * PAGE).sum())
    return DecodeBatch(attend.astype(np.int32), indptr, ids, slots.astype(np.int32), num_blocks,
                       meta={"shared_blocks": shared.astype(np.int32), "own_first": own_first,
                             "unique_tokens": unique, "prefix": prefix})


def pool_pressure_step(num_blocks: int, num_seqs: int, chunk: int, chunk_seqs: int,
                       rng: SplitMix64, budget: int | None = None) -> tuple[DecodeBatch, np.ndarray, np.ndarray]:
    """One step of a pool under pressure: `num_seqs` sequences with lengths
    ~LogNormal(ln 2048, 1) capped at 32,768 hold blocks drawn from a seeded
    permutation of a `num_blocks` pool. The first `chunk_seqs` are prefills
    in progress with `chunk` tokens of their prompt left; the engine's
    budget rule (PrefillAdder, inference-engine/src/prefill.rs:27-36,
    99-114, in the host library) gives each its chunk under `budget` prefill
    tokens (default chunk * chunk_seqs: every prefill finishes its prompt),
    and the others decode one token. Returns the decode batch of the
    decoding sequences, the chunk tokens' slots and all sequences' lengths
    before the step."""
    from .host import schedule_prefill_chunks

    lengths = np.asarray(lognormal_lengths(rng, num_seqs, 2048, 1.0, 32768), np.int64)
    chunks, _ = schedule_prefill_chunks(chunk * chunk_seqs if budget is None else budget, [chunk] * chunk_seqs)
    if 0 in chunks:
        raise ValueError("the budget leaves a prefill without a chunk this step")
    grow = np.ones(num_seqs, np.int64)
    grow[:chunk_seqs] = chunks
    nblk = (lengths + grow + PAGE - 1) // PAGE
    if int(nblk.sum()) > num_blocks:
        raise ValueError("the sequences need more blocks than the pool holds")
    perm = permutation(num_blocks, rng)
    starts = np.concatenate([[0], np.cumsum(nblk)])
    tables = [perm[starts[b]:starts[b + 1]] for b in range(num_seqs)]
    chunk_slots = []
    for b in range(chunk_seqs):
        pos = lengths[b] + np.arange(grow[b])
        chunk_slots.append(tables[b][pos // PAGE].astype(np.int64) * PAGE + pos % PAGE)
    dec = range(chunk_seqs, num_seqs)
    ctx = lengths[chunk_seqs:]
    indptr = np.zeros(len(dec) + 1, np.int32)
    np.cumsum(nblk[chunk_seqs:], out=indptr[1:])
    ids = np.concatenate([tables[b] for b in dec]).astype(np.int32)
    slots = ids[indptr[:-1] + ctx // PAGE].astype(np.int64) * PAGE + ctx % PAGE
    batch = DecodeBatch((ctx + 1).astype(np.int32), indptr, ids, slots.astype(np.int32), num_blocks)
    return batch, np.concatenate(chunk_slots).astype(np.int32), lengths.astype(np.int32)


# Benchmark configurations: the model shapes and batches the benchmarks are quoted on.
CONFIGS = {
    "qwen2.5-0.5b": dict(num_layers=24, num_q_heads=14, num_kv_heads=2, head_dim=64, dtype="f32",
                         batch=8, ctx_lo=32, ctx_hi=512, index=0),
    "qwen2.5-7b": dict(num_layers=28, num_q_heads=28, num_kv_heads=4, head_dim=128, dtype="bf16",
                       batch=64, ctx_lo=1024, ctx_hi=8192, index=1),
    "gemma-2b-mqa": dict(num_layers=18, num_q_heads=8, num_kv_heads=1, head_dim=256, dtype="bf16",
                         batch=128, ctx_lo=2048, ctx_hi=8192, index=2),
}


def config_batch(name: str, seed: int | None = None) -> DecodeBatch:
    c = CONFIGS[name]
    s = BASE_SEED + c["index"] if seed is None else seed
    rng = SplitMix64(s)
    ctx = uniform_contexts(c["batch"], c["ctx_lo"], c["ctx_hi"], rng)
    b = decode_batch_from_contexts(ctx, rng)
    b.seed = s
    return b


def algorithmic_bytes_attention(batch: DecodeBatch, num_q_heads: int, num_kv_heads: int,
                                head_dim: int, elem_bytes: int) -> int:
    """K+V read once + Q read + O written + block ids + context lengths."""
    kv = batch.total_tokens * 2 * num_kv_heads * head_dim * elem_bytes
    qo = 2 * batch.num_seqs * num_q_heads * head_dim * elem_bytes
    meta = 4 * int(batch.block_ids.size) + 4 * (batch.num_seqs + 1) + 4 * batch.num_seqs
    return kv + qo + meta


def algorithmic_bytes_append(num_tokens: int, num_kv_heads: int, head_dim: int,
                             elem_bytes: int) -> int:
    """K and V rows read and written + slot ids."""
    return 4 * num_tokens * num_kv_heads * head_dim * elem_bytes + 4 * num_tokens


def algorithmic_bytes_prep(num_tokens: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                           elem_bytes: int, rotary_dim: int, norm: bool) -> int:
    """Fused pre-attention step: q rows read (the q half of the gated
    projection) and written, k and v rows read and written, positions and
    slot ids, plus the norm weights and the frequency table."""
    rows = num_tokens * (2 * num_q_heads + 4 * num_kv_heads) * head_dim * elem_bytes
    return rows + 8 * num_tokens + (8 * head_dim if norm else 0) + 2 * rotary_dim


def tokens(rng: SplitMix64, n: int) -> np.ndarray:
    """n seeded token ids (u32, below 50,000)."""
    return np.asarray([rng.bounded(50_000) for _ in range(n)], np.uint32)


class RadixSharingScenario:
    """The radix-sharing configuration, phase by phase, on the host block
    manager (refcounted pool + radix tree), at Qwen2.5-7B shapes:

    1. `prefill_prefix()`: sequence 0 is admitted with a `prefix`-token prompt
       (4,100: 256 full blocks and a 4-token partial block), its K/V slots
       returned, and the prompt promoted into the radix tree
       (scheduler.rs:117, radix_cache.rs:287-294).
    2. `fork_and_suffixes()`: sequences 1..n-1 fork sequence 0 and share
       every prefix block, the partial one included; each then appends its
       own suffix ~U{suffix_lo..suffix_hi} (a prefill chunk). The first
       write into the shared partial block copies it (n - 1 copy pairs,
       returned); sequence 0, its last holder, writes in place. Every prompt
       (prefix + suffix) is then promoted.
    3. `decode_step()`: every sequence appends one token; returns the slots.
    4. `finish_and_evict()`: a third of the sequences finish (release: their
       promoted pages stay in the tree, the rest are freed), then LRU
       eviction of the tree (radix_cache.rs:243-282) until at least
       `evict_frac` of the live blocks are freed.
    5. `compaction()`: the block moves that pack the live blocks below the
       live count (tables and tree pages rewritten), for copy_blocks.

    Every result is a pure function of the seed."""

    def __init__(self, num_seqs: int = 256, prefix: int = 4100, suffix_lo: int = 64, suffix_hi: int = 1024,
                 decode_steps: int = 32, seed: int = BASE_SEED + 3, spare_blocks: int = 64):
        from .host import BlockManager

        rng = SplitMix64(seed)
        self.num_seqs, self.prefix, self.decode_steps = num_seqs, prefix, decode_steps
        self.suffix = [rng.uniform_int(suffix_lo, suffix_hi) for _ in range(num_seqs)]
        self.prefix_tokens = tokens(rng, prefix)
        self.prompts = [np.concatenate([self.prefix_tokens, tokens(rng, n)]) for n in self.suffix]
        full = prefix // PAGE
        part = prefix - full * PAGE
        own = [(part + n + decode_steps + PAGE - 1) // PAGE for n in self.suffix]
        self.num_blocks = full + sum(own) + spare_blocks
        self.bm = BlockManager(self.num_blocks)
        self.seqs = list(range(num_seqs))
        self.live = list(self.seqs)
        self.prefix_full_blocks = full

    def prefill_prefix(self) -> np.ndarray:
        bm = self.bm
        assert bm.admit(0, self.prefix_tokens) == 0
        slots, cow = bm.append(0, self.prefix)
        assert cow == []
        bm.promote(0, self.prefix_tokens)
        return slots.astype(np.int32)

    def fork_and_suffixes(self):
        """(cow_src, cow_dst, slots): the copies to run first, then the
        suffix tokens' slots in the order [1, .., n-1, 0]."""
        bm = self.bm
        for s in self.seqs[1:]:
            bm.fork(0, s)
        src, dst, slots = [], [], []
        for s in self.seqs[1:] + [0]:
            sl, cow = bm.append(s, self.suffix[s])
            slots.append(sl)
            for a, b in cow:
                src.append(a)
                dst.append(b)
        for s in self.seqs:
            bm.promote(s, self.prompts[s])
        return (np.asarray(src, np.int32), np.asarray(dst, np.int32),
                np.concatenate(slots).astype(np.int32))

    def decode_step(self) -> np.ndarray:
        return np.concatenate([self.bm.append(s, 1)[0] for s in self.live]).astype(np.int32)

    def finish_and_evict(self, evict_frac: float = 0.2):
        """(finished sequences, blocks freed, live blocks before)."""
        bm = self.bm
        done = self.seqs[::3]
        for s in done:
            bm.release(s)
        self.live = [s for s in self.seqs if s not in set(done)]
        live_before = bm.live_blocks()
        target = int(np.ceil(evict_frac * live_before))
        freed = 0
        while freed < target and bm.cached_pages() > 0:
            freed += bm.evict(max(1, min(256, target - freed)))
        return done, freed, live_before

    def compaction(self):
        return self.bm.plan_compaction()
