"""Decode-step benchmark of the paged-KV hot path on one MI355X.

One step = for every layer of the Qwen2.5-7B-shaped batch (28 layers, 28 query
heads, 4 KV heads, head_dim 128, bf16 KV, block size 16, 64 sequences with
context lengths uniform in [1024, 8192], block tables drawn from a seeded
permutation of the pool): append the step's K/V row of every sequence into its
slot, then run paged GQA decode attention over context + 1 tokens.

Prints one JSON line: whole-step HBM throughput in algorithmic bytes (K/V
read once, Q read, O written, appends read+written, block tables and slot
ids), tokens/s, the attention kernel's roofline fraction measured with HIP
events that the library records on its stream right before and after that
kernel (its split-K merge excluded; the whole layer's figure is nested
beside it) over the timed region, and the CPU baseline (the
oracle's reference-faithful restatement of the reference's CPU attention,
timed on a bounded sample on this host).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

The default run also measures the other configurations, each on its own
pool at full size, and nests their figures under "configs" (step time,
GB/s, % of peak, roofline, traffic source): the f32 Qwen2.5-0.5B step with
its block-table gather, the Gemma-2B MQA step, the radix-shared-prefix
scenario (its 32 decode steps, copy-on-write copies and compaction moves)
and the 200 GB pool-pressure step. `--no-configs` skips them.

`--op prep` measures the fused pre-attention kernel instead (q/k RMSNorm +
NeoX RoPE + K/V append, mkv_qk_norm_rope_append) on a prefill chunk of
`--tokens` tokens at the same head geometry, and prints its own JSON line.
`--op wire` measures the KV block wire format: export of `--handoff-blocks`
blocks (all layers) to a payload and its import into other blocks.
`--op gather` measures the block-table gather of the decode batch's contexts
(one layer per launch); `--op copy` measures copy_blocks (COW copies and
compaction moves) of `--copy-pairs` block pairs over all layers; `--op
extend` measures chunked-prefill attention (TFLOP/s against the bf16 MFMA
peak). `--op shared` measures the decode step of 256 sequences over one
radix-shared 4,100-token prefix (GB/s on unique and on logical bytes) and
its copy-on-write copies and compaction moves; `--op pressure` measures a
step of 8 chunk appends and 504 decodes over a 217,982-block (200 GB) pool.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import gc
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PREFILL_BUDGET = 4096  # prefill tokens per step of the pool-pressure configuration (max_prefill_tokens_per_iter)
METRIC = "paged KV append+decode-attn achieved HBM GB/s (% peak); decode tokens/s"

_HIP = None  # the HIP runtime torch loaded (ctypes), once a timing event is made


class _HipEvent:
    """HIP timing event created with hipEventDisableSystemFence: its record
    skips the system-scope release that a default event performs (an L2
    write-back and invalidate), which would slow the launches it brackets.
    Same calls as torch.cuda.Event: record(stream), elapsed_time(end) in ms
    after a synchronize."""

    def __init__(self, lib, handle):
        self._lib, self.handle = lib, handle

    def record(self, stream):
        rc = self._lib.hipEventRecord(self.handle, ctypes.c_void_p(stream.cuda_stream))
        if rc:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end) -> float:
        ms = ctypes.c_float()
        rc = self._lib.hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle)
        if rc:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        try:
            self._lib.hipEventDestroy(self.handle)
        except Exception:
            pass


def _event():
    """A timing event for the timed regions: _HipEvent, or torch's event where
    the runtime refuses the flag."""
    global _HIP
    import torch

    if _HIP is None:
        try:  # torch has loaded the runtime: this finds the same copy by its soname
            lib = ctypes.CDLL("libamdhip64.so.7")
            lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
            _HIP = lib
        except OSError:
            _HIP = False
    if _HIP:
        h = ctypes.c_void_p()
        if _HIP.hipEventCreateWithFlags(ctypes.byref(h), 0x20000000) == 0:  # hipEventDisableSystemFence
            return _HipEvent(_HIP, h)
    return torch.cuda.Event(enable_timing=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="qwen2.5-7b")
    ap.add_argument("--mode", choices=["step", "planned", "split"], default="step",
                    help="step: plan + fused append/attention per layer; planned: plan, append, "
                         "attention; split: append + split-grid attention")
    ap.add_argument("--pieces", type=int, default=0)
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--kernel", choices=["auto", "mfma", "valu"], default="auto")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="headline only: skip the other configurations' nested lines")
    ap.add_argument("--no-launch-events", action="store_true",
                    help="time the steps without per-launch HIP events (roofline fields null)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="about how long the CPU baseline's one-thread sample runs, per configuration")
    ap.add_argument("--op", choices=["decode", "prep", "wire", "gather", "copy", "append", "extend", "shared",
                                     "pressure", "small"],
                    default="decode",
                    help="decode: the decode step (headline); prep: the fused q/k-norm + RoPE + "
                         "append kernel on a prefill chunk; wire: KV block export + import of a "
                         "handoff; gather: block-table gather of the decode batch, one layer; "
                         "copy: copy_blocks of --copy-pairs block pairs, all layers; extend: chunked-"
                         "prefill attention of --extend-seqs chunks of --tokens-per-chunk after "
                         "--prefix tokens; shared: decode step of 256 sequences over a radix-shared "
                         "prefix, with its copy-on-write copies and compaction moves; pressure: "
                         "chunk appends + decode step over a 200 GB pool; small: latency-bound decode "
                         "steps of 1-12 sequences at Qwen2.5-7B heads")
    ap.add_argument("--extend-seqs", type=int, default=8, help="--op extend: sequences")
    ap.add_argument("--tokens-per-chunk", type=int, default=512, help="--op extend: chunk length")
    ap.add_argument("--prefix", type=int, default=4096, help="--op extend: cached tokens before the chunk")
    ap.add_argument("--copy-pairs", type=int, default=4096, help="--op copy: block pairs")
    ap.add_argument("--append-chunks", type=int, default=8,
                    help="--op append: 512-token chunks appended per launch (the pool-pressure step's 8)")
    ap.add_argument("--handoff-blocks", type=int, default=2048,
                    help="--op wire: blocks handed off (all layers)")
    ap.add_argument("--tokens", type=int, default=16384, help="--op prep: tokens in the chunk")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device to device (the known-size kernel that scales "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


def copy_calibration():
    """One 1 GiB device-to-device copy after a warm-up copy: the reference
    dispatch whose FETCH_SIZE and WRITE_SIZE counters, against its known
    2 x 1 GiB of traffic, give the scale factors of the HBM traffic figures."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n}), flush=True)


def profiled_traffic(key: str, field: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch from the committed rocprofv3 PMC summary of a
    workload (profiles/<key>_hbm_traffic.md: FETCH_SIZE and WRITE_SIZE,
    scaled by a 1 GiB copy kernel), or (None, None) when there is none.
    field: traffic_bytes_per_launch (the timed launch group) or
    traffic_bytes_per_kernel_launch (its dominant kernel alone)."""
    path = os.path.join(ROOT, "profiles", f"{key}_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(field + ":"):
                    return int(line.split(":", 1)[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def cpu_info():
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def _prefix_count(ctx, tokens: float) -> int:
    """Sequences taken from the front of the batch until their contexts hold
    about `tokens` tokens (at least one, at most all)."""
    c = np.cumsum(np.asarray(ctx, np.int64))
    return int(min(len(c), max(1, np.searchsorted(c, tokens, side="right"))))


def cpu_baseline(cfg, batch, step_bytes, budget_s: float = 8.0, paged=True):
    """Reference-faithful CPU decode (contiguous f32 cache grown by a copy per
    token, repeat_kv materialised, mask, softmax, matmuls) on a bounded sample
    of the step, scaled to a full step by its share of the step's tokens.

    The sample: a short calibration run gives the cost per token; then either
    every sequence for as many layer passes as about `budget_s` seconds allow,
    or, when one layer of the whole batch would take longer, the sequences at
    the front of the batch that fill about `budget_s` seconds of one layer.
    The primary figure is one thread, sequences one after another, as the
    reference executes requests serially
    (inference-backend/src/burn_backend.rs:44-71); the same kind of sample
    threaded over sequences on every host thread is reported beside it."""
    from oracle import oracle as orc

    ctx = np.asarray(batch.ctx_lens, np.int64)
    L, Hkv, Hq, D = cfg["num_layers"], cfg["num_kv_heads"], cfg["num_q_heads"], cfg["head_dim"]
    total_tok = int(ctx.sum())
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))

    def run(nseq: int, passes: int, nthreads: int, seed: int) -> float:
        orc.set_num_threads(nthreads)
        return sum(orc.ref_faithful_batch(ctx[:nseq], Hkv, Hq, D, seed=seed + 7919 * i) for i in range(passes))

    def sample(budget: float, nthreads: int, seed: int):
        """(sequences, layer passes, seconds, tokens) of one bounded sample."""
        ncal = _prefix_count(ctx, min(total_tok, 65536))
        per_tok = run(ncal, 1, nthreads, seed) / float(ctx[:ncal].sum())
        layer_s = per_tok * total_tok
        if layer_s <= budget:
            nseq, passes = len(ctx), int(max(1, min(2000, budget // max(layer_s, 1e-9))))
        else:
            nseq, passes = _prefix_count(ctx, budget / per_tok), 1
        t = run(nseq, passes, nthreads, seed + 1)
        return nseq, passes, t, int(ctx[:nseq].sum()) * passes

    orc.set_setup_threads(threads)  # the caches' seeded fill is set-up, outside the timed region
    n1, p1, t1, tok1 = sample(budget_s, 1, 1)
    step_1t = t1 * (total_tok * L) / tok1
    nn, pn, tn, tokn = sample(budget_s / 4, threads, 100)
    step_nt = tn * (total_tok * L) / tokn
    orc.set_num_threads(threads)
    orc.set_setup_threads(0)

    def what(nseq, passes, nthreads, t):
        seqs = f"all {len(ctx)} sequences" if nseq == len(ctx) else f"the first {nseq} of {len(ctx)} sequences"
        return (f"{passes} layer pass{'es' if passes > 1 else ''} of {seqs} ({nthreads} thread"
                f"{'s' if nthreads > 1 else ''}, {t:.1f} s), scaled by tokens to all {L} layers of the step")

    out = {
        "value": round(step_bytes / step_1t / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": what(n1, p1, 1, t1),
        "tokens_per_s": round(batch.num_seqs / step_1t, 2),
        "ms_per_step": round(step_1t * 1e3, 1),
        "threaded": {"value": round(step_bytes / step_nt / 1e9, 3), "unit": "GB/s", "cores": threads,
                     "tokens_per_s": round(batch.num_seqs / step_nt, 2), "ms_per_step": round(step_nt * 1e3, 1),
                     "sample": what(nn, pn, threads, tn)},
        "cpu_model": cpu_info(),
        "host_cpus": os.cpu_count(),
    }
    if not paged:
        return out
    # Second line: the efficient paged oracle (f32 accumulation over a bf16 /
    # f32 pool, threaded over sequences and heads) on one layer of the same
    # batch, K/V from a seeded host pool of the same blocks; scaled to a step.
    es = 2 if cfg["dtype"] == "bf16" else 4
    od = orc.desc(1, Hkv, D, batch.num_blocks, es)
    raw = np.random.default_rng(7).standard_normal(orc.pool_bytes(od) // es, dtype=np.float32)
    host = orc.f32_to_bf16(raw) if es == 2 else raw
    del raw
    q = np.random.default_rng(8).standard_normal((batch.num_seqs, Hq, D), dtype=np.float32)
    c0 = time.perf_counter()
    orc.decode_attention(od, host, 0, q, batch.block_indptr, batch.block_ids, batch.ctx_lens)
    tp = time.perf_counter() - c0
    del host
    step_p = tp * L
    out["paged_oracle"] = {"value": round(step_bytes / step_p / 1e9, 3), "unit": "GB/s", "cores": threads,
                           "tokens_per_s": round(batch.num_seqs / step_p, 2),
                           "sample": f"oracle paged decode attention, 1 layer of all {batch.num_seqs} sequences, "
                                     f"{threads} threads, {tp:.2f} s; scaled to a full step"}
    return out


def bench_prep(args):
    """The fused pre-attention kernel on one prefill chunk: `--tokens` tokens
    of one layer, q as the gated q_proj output [n, Hq, 2, D], RMSNorm(1 + w)
    on q and k, RoPE over the whole head (theta 1e6), k and v appended at the
    slots of freshly allocated blocks drawn from a seeded permutation of the
    pool. One launch per step; HIP events on the launch stream."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl
    from mitten_amd.device_pool import rope_inv_freq

    cfg = wl.CONFIGS[args.config]
    Hq, Hkv, D, dt = cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"], cfg["dtype"]
    n, rd = args.tokens, D
    nblocks = (n + 15) // 16 * 2
    desc = PoolDesc(1, Hkv, Hq, D, nblocks, dt)
    dev = torch.device("cuda:0")
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    rng = wl.SplitMix64(wl.BASE_SEED + 17)
    perm = wl.permutation(nblocks, rng)
    pos = np.arange(n, dtype=np.int64)
    slots = (perm[pos // 16].astype(np.int64) * 16 + pos % 16).astype(np.int32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl.BASE_SEED + 17)
    q = torch.randn((n, Hq, 2, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
    k = torch.randn((n, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
    v = torch.randn((n, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
    wq = (torch.rand(D, generator=gen, device=dev) - 0.5) * 0.2
    wk = (torch.rand(D, generator=gen, device=dev) - 0.5) * 0.2
    freq = torch.from_numpy(rope_inv_freq(rd, 1e6)).to(dev)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    pos_d, slots_d = i32(pos), i32(slots)
    out = torch.empty((n, Hq, D), dtype=tdt, device=dev)
    stream = torch.cuda.current_stream()
    launch_bytes = wl.algorithmic_bytes_prep(n, Hq, Hkv, D, desc.elem_bytes, rd, True)
    with DeviceKvPool(desc) as pool:
        def step():
            pool.qk_norm_rope_append(0, q, k, v, pos_d, slots_d, wq, wk, freq, eps=1e-6, out=out,
                                     stream=stream)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        pool.check()
        e0, e1 = _event(), _event()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        pool.check()
        # The engine's host form (mkv_qk_norm_rope_append_host): every layer
        # of a step passes the same host positions and slots, which are
        # staged once and then reused, so a call's host time stays flat
        # rather than waiting on the launch from a full staging ring earlier.
        layers = cfg["num_layers"]
        pos_h, slots_h = pos.astype(np.int32), slots.astype(np.uint32)
        # The first call allocates the staging slot. Python's collector stays
        # off while the calls are timed: a full collection in a process that
        # holds torch takes 35-43 ms and would land on one call at random.
        pool.qk_norm_rope_append(0, q, k, v, pos_h, slots_h, wq, wk, freq, eps=1e-6, out=out, stream=stream)
        torch.cuda.synchronize()
        enqueue = []
        gc.collect()
        gc.disable()
        h0, h1 = _event(), _event()
        h0.record(stream)
        for _ in range(args.steps):
            for _layer in range(layers):
                c0 = time.perf_counter()
                pool.qk_norm_rope_append(0, q, k, v, pos_h, slots_h, wq, wk, freq, eps=1e-6, out=out,
                                         stream=stream)
                enqueue.append(time.perf_counter() - c0)
        h1.record(stream)
        gc.enable()
        torch.cuda.synchronize()
        pool.check()
        host_launch_s = h0.elapsed_time(h1) / 1e3 / (args.steps * layers)
    launch_s = e0.elapsed_time(e1) / 1e3 / args.steps
    gbs = launch_bytes / launch_s / 1e9
    # CPU baseline: the oracle's restatement on a 2048-token sample.
    from oracle import oracle as orc

    sample = min(n, 2048)
    qh = np.random.default_rng(0).standard_normal((sample, Hq, D)).astype(np.float32)
    kh = np.random.default_rng(1).standard_normal((sample, Hkv, D)).astype(np.float32)
    wh = np.zeros(D, np.float32)
    fh = rope_inv_freq(rd, 1e6)
    c0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - c0 < 2.0 or reps == 0:
        orc.norm_rope_rows(qh, wh, 1e-6, fh, np.repeat(pos[:sample], Hq))
        orc.norm_rope_rows(kh, wh, 1e-6, fh, np.repeat(pos[:sample], Hkv))
        reps += 1
    cpu_s = (time.perf_counter() - c0) / reps
    cpu_gbs = wl.algorithmic_bytes_prep(sample, Hq, Hkv, D, desc.elem_bytes, rd, True) / cpu_s / 1e9
    print(json.dumps({
        "metric": "fused q/k RMSNorm + RoPE + K/V append achieved HBM GB/s",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(launch_s * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dt,
        "data": "synthetic: N(0,1) q/k/v from a seed; slots of a seeded block permutation",
        "config": {"workload": f"{args.config}-shaped prefill chunk, fused pre-attention step",
                   "tokens": n, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "rotary_dim": rd,
                   "q_layout": "gated [n, Hq, 2, D]", "norm": "RMSNorm(1 + w), eps 1e-6"},
        "tokens_per_s": round(n / launch_s, 1),
        "wall_ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "host_form": {"what": "mkv_qk_norm_rope_append_host with the same host positions and slots on each of a "
                              "step's layers, no synchronisation between calls, Python's collector off",
                      "layers_per_step": layers, "calls": len(enqueue),
                      "host_us_per_call_median": round(float(np.median(enqueue)) * 1e6, 1),
                      "host_us_per_call_max": round(max(enqueue) * 1e6, 1),
                      "gpu_us_per_call": round(host_launch_s * 1e6, 2)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "mkv_qk_norm_rope_append", "bytes_per_launch": launch_bytes,
                     "avg_launch_us": round(launch_s * 1e6, 2)},
        "cpu_baseline": {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"oracle norm + RoPE of {sample} tokens' q and k rows, f32, "
                                   f"{reps} repetitions"},
    }), flush=True)


def bench_wire(args):
    """A handoff of `--handoff-blocks` blocks of the config's pool (every
    layer, K and V): mkv_wire_export of blocks drawn from a seeded
    permutation into one payload with per-block checksums, then
    mkv_wire_import of that payload into other blocks with verification.
    One step = export + import; HIP events around each launch pair."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS[args.config]
    L, Hq, Hkv, D, dt = (cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                         cfg["dtype"])
    n = args.handoff_blocks
    nblocks = 2 * n + 64
    desc = PoolDesc(L, Hkv, Hq, D, nblocks, dt)
    dev = torch.device("cuda:0")
    rng = wl.SplitMix64(wl.BASE_SEED + 23)
    perm = wl.permutation(nblocks, rng)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    src, dst = i32(perm[:n]), i32(perm[n:2 * n])
    stream = torch.cuda.current_stream()
    with DeviceKvPool(desc) as pool:
        gen = torch.Generator(device=dev)
        gen.manual_seed(wl.BASE_SEED + 23)
        view = pool.tensor()
        for layer in range(L):
            view[layer].normal_(generator=gen)
        del view
        bb = pool.wire_block_bytes()
        payload = torch.empty(n * bb, dtype=torch.uint8, device=dev)
        sums = torch.empty(n, dtype=torch.int64, device=dev)
        got = torch.empty(n, dtype=torch.int64, device=dev)

        def step(ev=None):
            if ev:
                ev[0].record(stream)
            pool.wire_export(src, payload=payload, checksums=sums, stream=stream)
            if ev:
                ev[1].record(stream)
            pool.wire_import(dst, payload, expected=sums, checksums=got, stream=stream)
            if ev:
                ev[2].record(stream)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        pool.check()
        evs = [[_event() for _ in range(3)] for _ in range(args.steps)]
        t0 = time.perf_counter()
        for s_ in range(args.steps):
            step(evs[s_])
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        pool.check()
        exp_s = float(np.mean([e[0].elapsed_time(e[1]) for e in evs])) / 1e3
        imp_s = float(np.mean([e[1].elapsed_time(e[2]) for e in evs])) / 1e3
        # CPU baseline: the oracle's export of a 64-block sample of the same pool.
        from oracle import oracle as orc

        sample = min(n, 64)
        host = pool.read()
        od = orc.desc(L, Hkv, D, nblocks, desc.elem_bytes)
        ids_h = perm[:sample].astype(np.int32)
        c0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - c0 < 2.0 or reps == 0:
            orc.wire_export(od, host, ids_h, 0, L)
            reps += 1
        cpu_s = (time.perf_counter() - c0) / reps
    bytes_one = 2 * n * bb + 4 * n + 8 * n  # payload read + written, ids, checksums
    exp_gbs, imp_gbs = bytes_one / exp_s / 1e9, bytes_one / imp_s / 1e9
    step_gbs = 2 * bytes_one / (elapsed / args.steps) / 1e9
    print(json.dumps({
        "metric": "KV block wire export + import achieved HBM GB/s",
        "value": round(step_gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dt,
        "data": "synthetic: N(0,1) K/V in every block; block ids from a seeded permutation",
        "config": {"workload": f"{args.config}-shaped handoff of {n} blocks (all {L} layers, K and V)",
                   "blocks": n, "block_payload_bytes": bb, "payload_bytes": n * bb},
        "export": {"avg_launch_us": round(exp_s * 1e6, 2), "GB_s": round(exp_gbs, 2)},
        "import": {"avg_launch_us": round(imp_s * 1e6, 2), "GB_s": round(imp_gbs, 2),
                   "note": "includes the checksum compare launch"},
        "roofline": {"bound": "hbm", "achieved": round(exp_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(exp_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "mkv_wire_export (zero + wire_kernel<true>)", "bytes_per_launch": bytes_one,
                     "avg_launch_us": round(exp_s * 1e6, 2)},
        "cpu_baseline": {"value": round(2 * sample * bb / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1,
                         "kind": "port", "sample": f"oracle wire_export of {sample} blocks, {reps} repetitions"},
    }), flush=True)


def bench_move(args):
    """gather: the decode batch's block-table gather, one layer per launch,
    cycling over the layers (K and V of every context token read once through
    the block table and written contiguously). copy: copy_blocks of
    `--copy-pairs` (src, dst) pairs drawn from a seeded permutation of the
    pool, every layer, K and V. HIP events on the launch stream around each
    launch."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS[args.config]
    batch = wl.config_batch(args.config)
    L, Hq, Hkv, D, dt = (cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                         cfg["dtype"])
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    dev = torch.device("cuda:0")
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    stream = torch.cuda.current_stream()
    row = Hkv * D * desc.elem_bytes
    with DeviceKvPool(desc) as pool:
        gen = torch.Generator(device=dev)
        gen.manual_seed(batch.seed)
        view = pool.tensor()
        for layer in range(L):
            view[layer].normal_(generator=gen)
        del view
        if args.op == "gather":
            ctx = batch.ctx_lens.astype(np.int64)
            cptr = np.concatenate([[0], np.cumsum(ctx)]).astype(np.int32)
            tokens = int(cptr[-1])
            indptr, ids, ctx_indptr = i32(batch.block_indptr), i32(batch.block_ids), i32(cptr)
            n = tokens * Hkv * D
            tdt = torch.bfloat16 if dt == "bf16" else torch.float32
            out_k = torch.empty(n, dtype=tdt, device=dev)
            out_v = torch.empty(n, dtype=tdt, device=dev)
            launch_bytes = 4 * tokens * row + 4 * int(batch.block_ids.size) + 8 * (batch.num_seqs + 1)

            def launch(i):
                pool.gather(i % L, indptr, ids, ctx_indptr, int(ctx.max()), out_k=out_k, out_v=out_v,
                            total_tokens=tokens, stream=stream)
            kernel, what = "mkv_gather", (f"{args.config} decode batch: {batch.num_seqs} sequences, "
                                          f"{tokens} context tokens, one layer per launch")
        elif args.op == "copy":
            rng = wl.SplitMix64(batch.seed + 5)
            perm = wl.permutation(batch.num_blocks, rng)
            npairs = args.copy_pairs
            src, dst = i32(perm[:npairs]), i32(perm[npairs:2 * npairs])
            launch_bytes = 2 * npairs * L * 2 * desc.block_bytes + 8 * npairs

            def launch(i):
                pool.copy_blocks(src, dst, stream=stream)
            kernel, what = "mkv_copy_blocks", f"{args.config} pool: {npairs} block pairs, all {L} layers, K and V"
        elif args.op == "append":
            # The pool-pressure step's chunk appends: `--append-chunks` chunks
            # of 512 consecutive positions, each in 32 whole blocks drawn from
            # a seeded permutation of the pool; one layer per launch.
            rng = wl.SplitMix64(batch.seed + 6)
            perm = wl.permutation(batch.num_blocks, rng)
            nch = args.append_chunks
            blocks = perm[:nch * 32].astype(np.int64)
            slots_h = (blocks[:, None] * 16 + np.arange(16)[None, :]).reshape(-1).astype(np.uint32)
            n_tok = int(slots_h.size)
            tdt = torch.bfloat16 if dt == "bf16" else torch.float32
            kk = torch.randn((n_tok, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
            vv = torch.randn((n_tok, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
            slots_d = i32(slots_h.astype(np.int32))
            launch_bytes = 4 * n_tok * row + 4 * n_tok
            host_slots = args.mode == "planned"  # reuse --mode planned to select the host-slot entry point

            def launch(i):
                if host_slots:
                    pool.append(i % L, kk, vv, slots_h, stream=stream)
                else:
                    pool.append(i % L, kk, vv, slots_d, stream=stream)
            kernel = "mkv_append_host" if host_slots else "mkv_append"
            what = f"{args.config} pool: {nch} x 512-token chunk append ({n_tok} tokens), one layer per launch"
        for i in range(args.warmup):
            launch(i)
        torch.cuda.synchronize()
        pool.check()
        evs = [(_event(), _event())
               for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i, (a, b) in enumerate(evs):
            a.record(stream)
            launch(i)
            b.record(stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        pool.check()
        # CPU baseline: the oracle's gather (one sequence) or copy_blocks
        # (64 pairs) on this host, one thread.
        from oracle import oracle as orc

        host = pool.read()
        od = orc.desc(L, Hkv, D, batch.num_blocks, desc.elem_bytes)
        c0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - c0 < 2.0 or reps == 0:
            if args.op == "gather":  # 8 sequences: more than the host's caches hold
                ns = min(8, batch.num_seqs)
                hi = batch.block_indptr[ns]
                orc.gather(od, host, 0, batch.block_indptr[:ns + 1], batch.block_ids[:hi], batch.ctx_lens[:ns])
                cpu_bytes = 4 * int(batch.ctx_lens[:ns].sum()) * row
                sample = f"oracle gather of {ns} sequences ({int(batch.ctx_lens[:ns].sum())} tokens)"
            elif args.op == "copy":
                ps = min(64, npairs)
                orc.copy_blocks(od, host, perm[:ps], perm[npairs:npairs + ps])
                cpu_bytes = 2 * ps * L * 2 * desc.block_bytes
                sample = f"oracle copy_blocks of {ps} pairs, all layers"
            else:
                hk = host[0, 0, :n_tok // 16].reshape(n_tok, Hkv, D).copy()
                orc.append(od, host, 0, hk, hk, slots_h.astype(np.int32))
                cpu_bytes = launch_bytes
                sample = f"oracle append of the {n_tok} tokens, one layer"
            reps += 1
        cpu_s = (time.perf_counter() - c0) / reps
    launch_s = float(np.mean([a.elapsed_time(b) for a, b in evs])) / 1e3
    gbs = launch_bytes / launch_s / 1e9
    ref_copy = None
    if args.op == "append":  # a device copy of the same rows, as a floor for a launch of this size
        src = torch.cat([kk.reshape(-1), vv.reshape(-1)])
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        cevs = [(_event(), _event()) for _ in range(args.steps)]
        for a, b in cevs:
            a.record(stream)
            dst.copy_(src)
            b.record(stream)
        torch.cuda.synchronize()
        copy_s = float(np.mean([a.elapsed_time(b) for a, b in cevs])) / 1e3
        copy_bytes = 2 * src.numel() * src.element_size()
        ref_copy = {"what": "torch device copy of the same K/V rows (read + write)", "bytes": copy_bytes,
                    "avg_launch_us": round(copy_s * 1e6, 2), "GB_s": round(copy_bytes / copy_s / 1e9, 2)}
        del src, dst
    print(json.dumps({
        "metric": f"{kernel} achieved HBM GB/s",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dt,
        "data": "synthetic: N(0,1) K/V in every block; block tables / pairs from a seeded permutation",
        "config": {"workload": what, "op": args.op},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": kernel,
                     "bytes_per_launch": launch_bytes, "avg_launch_us": round(launch_s * 1e6, 2)},
        "cpu_baseline": {"value": round(cpu_bytes / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"{sample}, {reps} repetitions"},
        **({"reference_copy": ref_copy} if ref_copy else {}),
    }), flush=True)


PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X


def bench_extend(args):
    """Chunked-prefill attention of one layer at the config's head geometry:
    `--extend-seqs` sequences, each a chunk of `--tokens-per-chunk` new
    tokens after `--prefix` cached ones (the chunk's K/V already in the pool;
    block tables from a seeded permutation). FLOPs are the causal ones: a
    query at position p attends p + 1 keys, 4 * head_dim per (query head,
    key) for QK^T and PV."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS[args.config]
    Hq, Hkv, D = cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    B, n, prefix = args.extend_seqs, args.tokens_per_chunk, args.prefix
    ctx = [prefix + n] * B
    rng = wl.SplitMix64(wl.BASE_SEED + 31)
    batch = wl.decode_batch_from_contexts([c - 1 for c in ctx], rng)
    desc = PoolDesc(1, Hkv, Hq, D, batch.num_blocks, "bf16")
    dev = torch.device("cuda:0")
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    stream = torch.cuda.current_stream()
    with DeviceKvPool(desc) as pool:
        gen = torch.Generator(device=dev)
        gen.manual_seed(wl.BASE_SEED + 31)
        view = pool.tensor()
        view[0].normal_(generator=gen)
        del view
        q = torch.randn((B * n, Hq, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        out = torch.empty_like(q)
        qi, ip, ix, cl = (i32(np.arange(B + 1) * n), i32(batch.block_indptr), i32(batch.block_ids),
                          i32(batch.ctx_lens))

        def launch():
            pool.extend_attention(0, q, qi, ip, ix, cl, n, max(ctx), out=out, stream=stream)

        for _ in range(args.warmup):
            launch()
        torch.cuda.synchronize()
        pool.check()
        evs = [(_event(), _event())
               for _ in range(args.steps)]
        t0 = time.perf_counter()
        for a_, b_ in evs:
            a_.record(stream)
            launch()
            b_.record(stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        pool.check()
        # CPU baseline: the oracle's extend attention (f32, one thread) on the
        # last 32 tokens of the first sequence's chunk, timed on this host.
        from oracle import oracle as orc

        host = pool.read()
        od = orc.desc(1, Hkv, D, batch.num_blocks, 2)
        ns = min(n, 32)
        qs = orc.bf16_to_f32(q[n - ns:n].cpu().view(torch.int16).numpy().view(np.uint16))
        ind = batch.block_ids[batch.block_indptr[0]:batch.block_indptr[1]]
        c0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - c0 < 2.0 or reps == 0:
            orc.extend_attention(od, host, 0, qs, [0, ns], [0, ind.size], ind, [ctx[0]])
            reps += 1
        cpu_s = (time.perf_counter() - c0) / reps
    launch_s = float(np.mean([a_.elapsed_time(b_) for a_, b_ in evs])) / 1e3
    keys = B * sum(prefix + i + 1 for i in range(n))
    flops = 4.0 * D * Hq * keys
    cpu_flops = 4.0 * D * Hq * sum(ctx[0] - ns + i + 1 for i in range(ns))
    tf = flops / launch_s / 1e12
    kv_bytes = B * (prefix + n) * 2 * Hkv * D * 2
    print(json.dumps({
        "metric": "chunked-prefill (extend) attention achieved TFLOP/s",
        "value": round(tf, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V and Q from a seed; block tables from a seeded permutation",
        "config": {"workload": f"{args.config}-shaped extend attention, one layer", "sequences": B,
                   "chunk_tokens": n, "prefix_tokens": prefix, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D},
        "tokens_per_s": round(B * n / launch_s, 1),
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None, "kernel": "mkv_extend_attention",
                     "flops_per_launch": flops, "kv_bytes_once": kv_bytes,
                     "avg_launch_us": round(launch_s * 1e6, 2)},
        "cpu_baseline": {"value": round(cpu_flops / cpu_s / 1e12, 5), "unit": "TFLOP/s", "cores": 1,
                         "kind": "port", "sample": f"oracle extend attention (f32) of the last {ns} tokens of "
                                                   f"one {n}-token chunk after {prefix}, {reps} repetitions"},
    }), flush=True)


def _decode_step_run(pool, plan, batch, L, Hq, Hkv, D, seed, dev, stream, pre_layer=None, cached_loads=False):
    """Q and new K/V rows of every layer, and a step function: the host plan
    of the step (with its host page tables), then per layer `pre_layer(layer)`
    (if given) and the fused append + attention. step(events) records
    events[layer] before each layer and events[L] after the last."""
    import torch

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    B = batch.num_seqs
    q = torch.randn((L, B, Hq, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    kn = torch.randn((L, B, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    vn = torch.randn((L, B, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    out = torch.empty_like(q)
    ip, ix = batch.block_indptr.astype(np.uint32), batch.block_ids.astype(np.uint32)
    ctx_host = batch.ctx_lens.copy()
    plan.build(ctx_host, 0, stream=stream, block_indptr=ip, block_ids=ix)
    run_layer = pool.bind_decode_step(plan, kn, vn, q, None, None, out, stream=stream, cached_loads=cached_loads)

    def step(events=None):
        # The engine's per-step call: host page tables (u32 CSR) into the plan.
        plan.build(ctx_host, 0, stream=stream, block_indptr=ip, block_ids=ix)
        for layer in range(L):
            if events is not None:
                events[layer].record(stream)
            if pre_layer is not None:
                pre_layer(layer)
            run_layer(layer)
        if events is not None:
            events[L].record(stream)

    return step


def _time_steps(step, steps, warmup, stream, L=None, every=4, before_pass=None):
    """Wall-clock seconds per step over `steps` steps after `warmup`, with no
    event recorded inside them; then a second pass of `steps` steps with an
    event pair around each step gives the HIP-event average of one step on
    `stream`, and (with L) per-layer events on every `every`-th step of that
    pass the average of one layer's bracket. before_pass(): called before
    each pass (a workload that cycles through its steps' metadata restarts)."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if before_pass:
        before_pass()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    evs = [(_event(), _event()) for _ in range(steps)]
    lay = {i: [_event() for _ in range(L + 1)]
           for i in range(0, steps, every)} if L else {}
    if before_pass:
        before_pass()
    for i, (a_, b_) in enumerate(evs):
        a_.record(stream)
        if L:
            step(lay.get(i))
        else:
            step()
        b_.record(stream)
    torch.cuda.synchronize()
    ev = float(np.mean([a_.elapsed_time(b_) for a_, b_ in evs])) / 1e3
    if not L:
        return wall, ev
    layer_s = float(np.mean([e[j].elapsed_time(e[j + 1]) for e in lay.values() for j in range(L)])) / 1e3
    return wall, ev, layer_s


def _time_copies(pool, src, dst, reps, stream):
    """HIP-event average seconds of one copy_blocks launch of the pairs:
    (the kernel alone, from device int32 pair arrays (mkv_copy_blocks);
    the engine's host call: u32 pairs validated, uploaded and launched
    (mkv_copy_blocks_host), its upload inside the bracket)."""
    import torch

    s_, d_ = np.ascontiguousarray(src, np.uint32), np.ascontiguousarray(dst, np.uint32)
    sd = torch.from_numpy(s_.astype(np.int32)).to(stream.device)
    dd = torch.from_numpy(d_.astype(np.int32)).to(stream.device)
    out = []
    for host in (False, True):
        call = (lambda: pool.copy_blocks(s_, d_, stream=stream)) if host else \
            (lambda: pool.copy_blocks(sd, dd, stream=stream))
        # One call per slot of the library's host staging ring first: a slot is
        # allocated (or grown) at its first use at a size, as in an engine's
        # first steps, not in its steady state.
        for _ in range(9 if host else 1):
            call()
        torch.cuda.synchronize()
        evs = [(_event(), _event()) for _ in range(reps)]
        for a_, b_ in evs:
            a_.record(stream)
            call()
            b_.record(stream)
        torch.cuda.synchronize()
        pool.check()
        out.append(float(np.mean([a_.elapsed_time(b_) for a_, b_ in evs])) / 1e3)
    return out[0], out[1]


def bench_shared(steps, warmup, cpu=True, compare_whole=True, cpu_seconds=8.0):
    """The radix-sharing configuration, driven by the host block manager
    (wl.RadixSharingScenario) at Qwen2.5-7B shapes, all 28 layers: 256
    sequences share a 4,100-token prefix (255 copy-on-write copies of its
    partial block, timed as one copy_blocks launch over all layers), append
    suffixes ~U{64..1024}, then run the configuration's 32 decode steps, each
    with its own tables from the block manager: the plan holds the step's
    host tables split at the shared prefix (mkv_decode_plan_build_shared_prefix)
    and every layer runs mkv_decode_step_shared_prefix (the prefix read once
    for all sequences on MFMA tiles, the suffixes through the plan, merged)
    with the fused append. After them a third of the sequences finish, LRU
    eviction frees 20% of the blocks and the compaction's block moves (from
    the block manager's plan) are timed as one copy_blocks launch. GB/s is
    on unique bytes (each shared block counted once: the HBM figure) and on
    logical bytes (each sequence's whole context). `steps` is ignored: the
    configuration's 32 decode steps are the timed steps."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS["qwen2.5-7b"]
    L, Hq, Hkv, D = cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    sc = wl.RadixSharingScenario()
    bm, B = sc.bm, sc.num_seqs
    desc = PoolDesc(L, Hkv, Hq, D, sc.num_blocks, "bf16")
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    row = 2 * Hkv * D * 2  # K and V bytes of one token in one layer
    per_pair = L * 2 * 16 * Hkv * D * 2 * 2 + 8
    with DeviceKvPool(desc) as pool:
        gen = torch.Generator(device=dev)
        gen.manual_seed(wl.BASE_SEED + 3)
        view = pool.tensor()
        for layer in range(L):  # N(0,1) K/V in every slot (the prefill's contents)
            view[layer].normal_(generator=gen)
        del view
        sc.prefill_prefix()
        cow_src, cow_dst, _ = sc.fork_and_suffixes()
        cow_s, cow_host_s = _time_copies(pool, cow_src, cow_dst, 10, stream)
        # The 32 decode steps' metadata, from the block manager.
        metas = []
        for _ in range(sc.decode_steps):
            sc.decode_step()
            ip, ids, ctx = bm.batch(sc.seqs)
            pre, sptr, sids, slen = bm.batch_shared_prefix(sc.seqs)
            shared_tok = 16 * int(pre.size)
            unique_tok = int(ctx.sum()) - (B - 1) * shared_tok
            metas.append(dict(ip=ip, ids=ids, ctx=ctx, pre=pre.astype(np.uint32), sptr=sptr.astype(np.uint32),
                              sids=sids.astype(np.uint32), slen=slen, unique_tok=unique_tok))
        gen2 = torch.Generator(device=dev)
        gen2.manual_seed(wl.BASE_SEED + 33)
        bf = lambda *shape: torch.randn(shape, generator=gen2, device=dev, dtype=torch.float32).to(torch.bfloat16)
        q, kn, vn = bf(L, B, Hq, D), bf(L, B, Hkv, D), bf(L, B, Hkv, D)
        out = torch.empty_like(q)
        m0 = metas[0]
        splan = pool.plan_shared_prefix(m0["pre"], m0["slen"], m0["sptr"], m0["sids"], stream=stream)
        run_sp = pool.bind_decode_step_shared_prefix(splan, kn, vn, q, None, None, None, out, stream=stream)
        cursor = [0]

        def step(events=None):
            m = metas[cursor[0] % len(metas)]
            cursor[0] += 1
            splan.build(m["slen"], 0, stream=stream, block_indptr=m["sptr"], block_ids=m["sids"],
                        prefix_ids=m["pre"])
            for layer in range(L):
                if events is not None:
                    events[layer].record(stream)
                run_sp(layer)
            if events is not None:
                events[L].record(stream)

        for _ in range(warmup):  # the first step's metadata, rewritten by the timed first step
            cursor[0] = 0
            step()
        wall, ev_step, layer_s = _time_steps(step, len(metas), 0, stream, L=L,
                                             before_pass=lambda: cursor.__setitem__(0, 0))
        pool.check()
        info = splan.info()
        splan.close()
        qo_meta = 2 * B * Hq * D * 2 + 4 * (B + 1) + 4 * B
        app = wl.algorithmic_bytes_append(B, Hkv, D, 2)
        unique = float(np.mean([L * (m["unique_tok"] * row + qo_meta + 4 * int(m["sids"].size + m["pre"].size) + app)
                                for m in metas]))
        logical = float(np.mean([L * (int(m["ctx"].sum()) * row + qo_meta + 4 * int(m["ids"].size) + app)
                                 for m in metas]))
        compare = None
        if compare_whole:  # the same last step through mkv_decode_step over the whole tables
            last = metas[-1]
            plan = pool.plan(last["ctx"], stream=stream, block_indptr=last["ip"].astype(np.uint32),
                             block_ids=last["ids"].astype(np.uint32))
            lb = wl.DecodeBatch(last["ctx"], last["ip"], last["ids"], np.zeros(B, np.int32), sc.num_blocks)
            step_c = _decode_step_run(pool, plan, lb, L, Hq, Hkv, D, wl.BASE_SEED + 33, dev, stream, cached_loads=True)
            wall_c, _ = _time_steps(step_c, 8, 2, stream)
            step_nt = _decode_step_run(pool, plan, lb, L, Hq, Hkv, D, wl.BASE_SEED + 33, dev, stream)
            wall_nt, _ = _time_steps(step_nt, 8, 2, stream)
            plan.close()
            pool.check()
            compare = {"whole_tables_cached_loads": {"entry": "mkv_decode_step, MKV_ATTN_CACHED_LOADS",
                                                     "ms_per_step": round(wall_c * 1e3, 4)},
                       "whole_tables_nontemporal": {"entry": "mkv_decode_step", "ms_per_step": round(wall_nt * 1e3, 4)}}
        # A third of the sequences finish, eviction frees 20% of the blocks,
        # and the compaction's moves pack the pool.
        done, freed, live_before = sc.finish_and_evict()
        mv_src, mv_dst = sc.compaction()
        mv_s, mv_host_s = _time_copies(pool, mv_src, mv_dst, 10, stream)
        bm.check_invariants()
    layer_unique = unique / L
    result = {
        "metric": "shared-prefix decode step: HBM GB/s on unique bytes (% peak); effective GB/s on logical bytes",
        "value": round(unique / wall / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": len(metas),
        "warmup": warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V/Q from a seed; tables from the host block manager (fork, copy-on-write, "
                "growth, eviction, compaction)",
        "config": {"workload": f"radix-shared decode: {B} sequences over one {sc.prefix}-token prefix (suffixes "
                               f"U[64, 1024]), {sc.decode_steps} decode steps, Qwen2.5-7B heads, {L} layers",
                   "layers": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block_size": 16,
                   "sequences": B, "prefix_tokens": sc.prefix, "shared_blocks": int(metas[0]["pre"].size),
                   "pool_blocks": sc.num_blocks, "plan": info,
                   "metadata": "host page tables split at the shared prefix, held by the step's plan"},
        "pct_peak": round(100.0 * unique / wall / 1e9 / PEAK_HBM_GBS, 2),
        "effective_gbs_logical": round(logical / wall / 1e9, 2),
        "logical_bytes_per_step": int(logical), "unique_bytes_per_step": int(unique),
        "tokens_per_s": round(B / wall, 1),
        "step_us_hip_events": round(ev_step * 1e6, 1),
        "roofline": {"bound": "hbm", "achieved": round(layer_unique / layer_s / 1e9, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(layer_unique / layer_s / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("decode_step_radix_shared_prefix_qwen2.5-7b")[0],
                     "traffic_source": profiled_traffic("decode_step_radix_shared_prefix_qwen2.5-7b")[1],
                     "kernel": "mkv_decode_step_shared_prefix (prefix tiles + suffix plan + merge, per layer)",
                     "bytes_per_launch": int(layer_unique), "avg_launch_us": round(layer_s * 1e6, 2)},
        "entry": "mkv_decode_step_shared_prefix (prefix once on MFMA tiles, suffix plan, merge)",
        "cow_copies": {"pairs": int(cow_src.size), "bytes": int(cow_src.size) * per_pair,
                       "avg_launch_us": round(cow_s * 1e6, 2),
                       "gbs": round(cow_src.size * per_pair / cow_s / 1e9, 2),
                       "host_call_us": round(cow_host_s * 1e6, 2),
                       "timing": "avg_launch_us: the kernel from device pair arrays; host_call_us: "
                                 "mkv_copy_blocks_host (u32 pairs checked, uploaded, launched)"},
        "compaction_moves": {"pairs": int(mv_src.size), "bytes": int(mv_src.size) * per_pair,
                             "finished_sequences": len(done), "blocks_freed_by_eviction": int(freed),
                             "live_blocks_before": int(live_before),
                             "avg_launch_us": round(mv_s * 1e6, 2),
                             "gbs": round(mv_src.size * per_pair / mv_s / 1e9, 2),
                             "host_call_us": round(mv_host_s * 1e6, 2)},
        "cpu_baseline": None,
        "timing": ("value and ms_per_step: the 32 steps, no event recorded inside them; roofline: a second "
                   "pass of the 32 steps with per-layer events on every fourth"),
    }
    if compare:
        result.update(compare)
    if cpu:
        last = metas[-1]
        lb = wl.DecodeBatch(last["ctx"], last["ip"], last["ids"], np.zeros(B, np.int32), sc.num_blocks)
        result["cpu_baseline"] = cpu_baseline(cfg, lb, logical, cpu_seconds)
        result["cpu_baseline"]["bytes"] = "logical (each sequence's whole context)"
    torch.cuda.empty_cache()
    return result


def bench_pressure(steps, warmup, cpu=True, cpu_seconds=8.0):
    """One step of a pool under pressure (the pool-pressure configuration):
    the 217,982-block pool of a 200 GB budget (all 28 layers, Qwen2.5-7B
    heads), 512 sequences with log-normal lengths (median 2,048, sigma 1,
    capped at 32,768) in blocks from a seeded permutation of the pool. Eight
    prefills in progress have a 512-token chunk of their prompt left; the
    engine's budget rule (PrefillAdder, 4,096 prefill tokens per step) gives
    each its chunk. Per step and layer, the 8 append their chunk
    (mkv_append_host: host u32 slots, the same for every layer, so uploaded
    once per step) and the other 504 run
    the fused append + decode attention from a plan holding the step's host
    tables; the chunks' prefill attention is left out, as the configuration
    states."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS["qwen2.5-7b"]
    L, Hq, Hkv, D = cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    nblocks, seqs, chunk, chunk_seqs = 217_982, 512, 512, 8
    batch, chunk_slots, lengths = wl.pool_pressure_step(nblocks, seqs, chunk, chunk_seqs,
                                                        wl.SplitMix64(wl.BASE_SEED + 4), budget=PREFILL_BUDGET)
    desc = PoolDesc(L, Hkv, Hq, D, nblocks, "bf16")
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    n_chunk = int(chunk_slots.size)
    step_bytes = L * (wl.algorithmic_bytes_attention(batch, Hq, Hkv, D, 2)
                      + wl.algorithmic_bytes_append(batch.num_seqs, Hkv, D, 2)
                      + wl.algorithmic_bytes_append(n_chunk, Hkv, D, 2))
    with DeviceKvPool(desc) as pool:
        gen = torch.Generator(device=dev)
        gen.manual_seed(wl.BASE_SEED + 4)
        view = pool.tensor()
        for layer in range(L):
            view[layer].normal_(generator=gen)
        del view
        kc = torch.randn((L, n_chunk, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        vc = torch.randn((L, n_chunk, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
        cs = chunk_slots.astype(np.uint32)

        def chunk_append(layer):
            pool.append(layer, kc[layer], vc[layer], cs, stream=stream)

        plan = pool.plan(batch.ctx_lens, stream=stream)
        step = _decode_step_run(pool, plan, batch, L, Hq, Hkv, D, wl.BASE_SEED + 44, dev, stream,
                                pre_layer=chunk_append)
        wall, ev, layer_s = _time_steps(step, steps, warmup, stream, L=L)
        pool.check()
        info = plan.info()
        plan.close()
        pool_bytes = pool.nbytes
        del kc, vc
    result = {
        "metric": "pool-pressure step (chunk appends + fused decode step): achieved HBM GB/s (% peak)",
        "value": round(step_bytes / wall / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V/Q from a seed; log-normal lengths and block ids from a seeded permutation",
        "config": {"workload": f"pool-pressure step: {nblocks}-block pool ({pool_bytes / 1e9:.1f} GB), {seqs} "
                               f"log-normal sequences, {chunk_seqs} x {chunk}-token chunk appends + "
                               f"{batch.num_seqs} decodes, Qwen2.5-7B heads, {L} layers",
                   "layers": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block_size": 16,
                   "pool_blocks": nblocks, "pool_bytes": pool_bytes, "sequences": seqs,
                   "tokens_held": int(lengths.sum()), "decode_sequences": batch.num_seqs,
                   "tokens_attended": batch.total_tokens, "chunk_tokens": n_chunk, "plan": info,
                   "metadata": "host u32 chunk slots per append; host page tables held by the step's plan"},
        "pct_peak": round(100.0 * step_bytes / wall / 1e9 / PEAK_HBM_GBS, 2),
        "step_bytes": step_bytes, "tokens_per_s": round(batch.num_seqs / wall, 1),
        "tokens_per_s_what": "decode tokens/s: the step's decoding sequences / step time (the chunks' tokens "
                             "are appended, not decoded)",
        "chunk_tokens_per_s": round(n_chunk / wall, 1),
        "step_us_hip_events": round(ev * 1e6, 1),
        "roofline": {"bound": "hbm", "achieved": round(step_bytes / L / layer_s / 1e9, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(step_bytes / L / layer_s / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("pool_pressure_step_qwen2.5-7b")[0],
                     "traffic_source": profiled_traffic("pool_pressure_step_qwen2.5-7b")[1],
                     "kernel": "mkv_append_host (chunks) + mkv_decode_step (per layer)",
                     "bytes_per_launch": step_bytes // L, "avg_launch_us": round(layer_s * 1e6, 2)},
        "cpu_baseline": None,
        "timing": ("value and ms_per_step: the K timed steps, no event recorded inside them; roofline: a "
                   "second pass of K steps with per-layer events on every fourth"),
    }
    if cpu:
        result["cpu_baseline"] = cpu_baseline(cfg, batch, step_bytes, cpu_seconds, paged=False)
    torch.cuda.empty_cache()
    return result


def decode_config(name: str, steps: int, warmup: int, mode: str = "step", pieces: int = 0,
                  kernel: str | None = None, split_tokens: int = 0, launch_events: bool = True):
    """One decode-step configuration (wl.CONFIGS[name]) on a fresh pool.
    A step is, per layer: append of every sequence's new K/V row + paged
    decode attention (`mode` step: one fused mkv_decode_step per layer from a
    plan holding the step's host page tables; planned: mkv_append +
    mkv_decode_attention_planned; split: mkv_append + mkv_decode_attention).
    The f32 Qwen2.5-0.5B configuration also gathers every layer's block
    tables into contiguous per-sequence caches, as its step states: in step
    mode inside the step (mkv_decode_step_gather), otherwise by
    mkv_gather_host after it. Returns (result dict, batch, step_bytes); the
    pool is freed."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS[name]
    batch = wl.config_batch(name)
    L, Hq, Hkv, D, dt = cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"], cfg["dtype"]
    B = batch.num_seqs
    with_gather = name == "qwen2.5-0.5b"
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, dt)
    dev = torch.device("cuda:0")
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    es = desc.elem_bytes

    pool = DeviceKvPool(desc)
    gen = torch.Generator(device=dev)
    gen.manual_seed(batch.seed)
    view = pool.tensor()
    for layer in range(L):  # N(0,1) K/V in every slot, one layer at a time
        view[layer].normal_(generator=gen)
    del view
    q = torch.randn((L, B, Hq, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
    k_new = torch.randn((L, B, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
    v_new = torch.randn((L, B, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(tdt)
    out = torch.empty_like(q)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    indptr, ids, ctx, slots = (i32(batch.block_indptr), i32(batch.block_ids), i32(batch.ctx_lens),
                               i32(batch.slot_mapping))
    max_ctx = batch.max_ctx
    ws = torch.empty(max(1, pool.workspace_size(B, max_ctx, split_tokens)), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    gk = torch.empty(batch.total_tokens * Hkv * D, dtype=tdt, device=dev) if with_gather else None
    gv = torch.empty_like(gk) if with_gather else None

    attn_bytes = wl.algorithmic_bytes_attention(batch, Hq, Hkv, D, es)
    app_bytes = wl.algorithmic_bytes_append(B, Hkv, D, es)
    # The gather reads every row and writes it back contiguous; fused into the
    # step (f32 step mode) it reads nothing the attention does not already.
    fused_gather = with_gather and mode == "step"
    gather_bytes = (0 if not with_gather else 2 * batch.total_tokens * Hkv * D * es if fused_gather
                    else 4 * batch.total_tokens * Hkv * D * es + 4 * int(batch.block_ids.size))
    step_bytes = L * (attn_bytes + app_bytes + gather_bytes)
    # Bytes of the work the HIP events bracket per layer: the fused step moves
    # the append's bytes too, and the gather follows it in the same bracket.
    launch_bytes = attn_bytes + (app_bytes if mode == "step" else 0) + gather_bytes

    ctx_host = batch.ctx_lens.copy()
    ip_h, ids_h = batch.block_indptr.astype(np.uint32), batch.block_ids.astype(np.uint32)
    plan = pool.plan(ctx_host, pieces=pieces, stream=stream, block_indptr=ip_h, block_ids=ids_h)

    # The f32 configuration's gather goes with each layer's step: the
    # per-head kernel stores the rows as it reads them (mkv_decode_step_gather).
    run_layer = pool.bind_decode_step(plan, k_new, v_new, q, None, None, out, kernel=kernel, stream=stream,
                                      gather_out=(gk, gv) if fused_gather else None)

    def step(events=None, kevents=None):
        """events: None, or L+1 timing events recorded between layers;
        kevents: None, or per layer a (start, end) pair that the library
        records around the layer's attention kernel alone."""
        if mode != "split":
            # The engine's one call per step: host lengths and host page
            # tables (u32 CSR), validated, copied and uploaded with the plan.
            plan.build(ctx_host, pieces, stream=stream, block_indptr=ip_h, block_ids=ids_h)
        for layer in range(L):
            if mode != "step":
                pool.append(layer, k_new[layer], v_new[layer], slots, stream=stream)
            if events is not None:
                events[layer].record(stream)
            if kevents is not None and kevents[layer] is not None:
                pool.set_launch_events(*kevents[layer])
            if mode == "step":
                run_layer(layer)
            elif mode == "planned":
                pool.decode_attention_planned(layer, plan, q[layer], None, None, out=out[layer],
                                              kernel=kernel, stream=stream)
            else:
                pool.decode_attention(layer, q[layer], indptr, ids, ctx, max_ctx, out=out[layer],
                                      split_tokens=split_tokens, workspace=ws, kernel=kernel,
                                      stream=stream)
            if with_gather and not fused_gather:
                pool.gather_host(layer, ip_h, ids_h, ctx_host, out_k=gk, out_v=gv, stream=stream)
        if events is not None:
            events[L].record(stream)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    pool.check()

    # Launch timing, in a pass after the timed steps: an event chain around
    # every layer's launch on every EVENT_EVERY-th step of that pass (events
    # cost GPU time; sampling keeps those steps close to unperturbed).
    # The planned modes also time the attention kernel alone (the library
    # records a pair of events around it, before its merge) on every fourth
    # layer of the steps in between, a different quarter of the layers each
    # time. (A pair on every layer of those steps, on top of the layer
    # events, made the runtime stall the host for about 30 ms once per run.)
    EVENT_EVERY = 4
    timed = [s_ for s_ in range(steps) if s_ % EVENT_EVERY == 0 and launch_events]
    ev = {s_: [_event() for _ in range(L + 1)] for s_ in timed}
    ktimed = [s_ for s_ in range(steps) if s_ % EVENT_EVERY == 2 and launch_events and mode != "split"]
    kev = {s_: [(_event(), _event()) if layer % 4 == (s_ // EVENT_EVERY) % 4 else None for layer in range(L)]
           for s_ in ktimed}
    for pairs in kev.values():
        for pair in pairs:
            if pair is not None and not isinstance(pair[0], _HipEvent):  # torch creates its event at the first record
                pair[0].record(stream)
                pair[1].record(stream)
    torch.cuda.synchronize()
    # The timed steps record no event: `value` comes from unperturbed steps.
    t0 = time.perf_counter()
    for s_ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    pool.check()
    elapsed = t1 - t0
    # A second pass of as many steps carries the sampled events that time
    # the layers and the attention kernel (the roofline's figures).
    if ev or kev:
        for s_ in range(steps):
            step(ev.get(s_), kev.get(s_))
        torch.cuda.synchronize()
        pool.check()
    ms_step = elapsed / steps * 1e3
    attn_ms = [e[i].elapsed_time(e[i + 1]) for e in ev.values() for i in range(L)] or [float("nan")]
    attn_avg_s = float(np.mean(attn_ms)) / 1e3
    gbs = step_bytes / (elapsed / steps) / 1e9
    attn_gbs = launch_bytes / attn_avg_s / 1e9
    # The dominant kernel alone: attention (with the fused append in step
    # mode), its merge and the gather excluded.
    kern_bytes = attn_bytes + (app_bytes if mode == "step" else 0) + (gather_bytes if fused_gather else 0)
    kern_ms = [k[i][0].elapsed_time(k[i][1]) for k in kev.values() for i in range(L) if k[i] is not None]
    kern_avg_s = float(np.mean(kern_ms)) / 1e3 if kern_ms else float("nan")
    kern_gbs = kern_bytes / kern_avg_s / 1e9 if kern_ms else float("nan")
    traffic, traffic_src = profiled_traffic(f"decode_{mode}_{name}")
    kernel_name = {"step": "mkv_decode_step (append + attention + merge, per layer)",
                   "planned": "mkv_decode_attention_planned (attention + merge, per layer)",
                   "split": "mkv_decode_attention (attention + merge, per layer)"}[mode]
    if fused_gather:
        kernel_name = "mkv_decode_step_gather (append + attention + gather + merge, per layer)"
    elif with_gather:
        kernel_name += " + mkv_gather_host"
    layer = {"what": kernel_name, "bytes": launch_bytes, "avg_us": round(attn_avg_s * 1e6, 2),
             "GB_s": round(attn_gbs, 2), "frac": round(attn_gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
             "launches_timed": len(attn_ms) if ev else 0}
    if kern_ms:
        # The roofline of the dominant kernel: the attention kernel alone.
        ktraffic, _ = profiled_traffic(f"decode_{mode}_{name}", "traffic_bytes_per_kernel_launch")
        roof = {"bound": "hbm", "achieved": round(kern_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(kern_gbs / PEAK_HBM_GBS, 4), "traffic": ktraffic, "traffic_source": traffic_src,
                "kernel": "the decode attention kernel alone" + (" (with the fused append)" if mode == "step" else "")
                          + (" and gather" if fused_gather else "")
                          + ", timed by events the library records around it",
                "bytes_per_launch": kern_bytes, "avg_launch_us": round(kern_avg_s * 1e6, 2),
                "launches_timed": len(kern_ms), "layer": layer}
    else:
        roof = {"bound": "hbm", "achieved": round(attn_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(attn_gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "kernel": kernel_name, "bytes_per_launch": launch_bytes, "avg_launch_us": round(attn_avg_s * 1e6, 2),
                "launches_timed": len(attn_ms) if ev else 0}
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic: N(0,1) K/V/Q from a seed; block tables from a seeded permutation of the pool",
        "config": {"workload": f"{name} decode step (append + paged decode attention per layer"
                               + (" + block-table gather" if with_gather else "") + ")",
                   "layers": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block_size": 16,
                   "sequences": B, "ctx_range": [cfg["ctx_lo"], cfg["ctx_hi"]],
                   "tokens_attended": batch.total_tokens, "pool_blocks": batch.num_blocks,
                   "pool_bytes": pool.nbytes, "seed": batch.seed, "mode": mode,
                   "plan": plan.info(), "split_tokens": split_tokens, "kernel": kernel or "auto",
                   "metadata": "host page tables (u32 CSR) held by the step's plan"},
        "pct_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "tokens_per_s": round(B / (elapsed / steps), 1),
        "step_bytes": step_bytes,
        "roofline": roof,
        "cpu_baseline": None,
        "timing": ("value and ms_per_step: the K timed steps, no event recorded inside them; roofline: a "
                   "second pass of K steps with sampled launch events"),
    }
    plan.close()
    pool.close()
    del q, k_new, v_new, out, ws, gk, gv
    torch.cuda.empty_cache()
    return result, batch, step_bytes


def _nested(r: dict) -> dict:
    """The fields of a configuration's result kept in the headline line."""
    keep = ("metric", "value", "unit", "ms_per_step", "pct_peak", "tokens_per_s", "tokens_per_s_what",
            "chunk_tokens_per_s", "steps", "warmup", "dtype", "config", "roofline", "effective_gbs_logical",
            "step_bytes", "unique_bytes_per_step", "logical_bytes_per_step", "cow_copies", "compaction_moves",
            "cpu_baseline", "timing")
    return {k: r[k] for k in keep if k in r}


SMALL_BATCHES = [[4096], [8192], [4096] * 4, [2048] * 8, [8192] * 4, [4096] * 12, [8192] * 8]


def bench_small(args):
    """Decode steps of batches too small to fill the device (1-12 sequences
    at Qwen2.5-7B heads, bf16; 8 x 8k is the first that fills it): the fused append + attention per layer from a
    plan holding the host tables, as in the headline step. Latency-bound, so
    the figure is microseconds per layer; each batch also reports its K/V
    bytes at that time."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS["qwen2.5-7b"]
    L, Hq, Hkv, D = 4, cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    dev = torch.device("cuda:0")
    rows = []
    for ctxs in SMALL_BATCHES:
        batch = wl.decode_batch_from_contexts([c - 1 for c in ctxs], wl.SplitMix64(wl.BASE_SEED + 31),
                                              extra_blocks=2)
        desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, "bf16")
        B = len(ctxs)
        gen = torch.Generator(device=dev)
        gen.manual_seed(wl.BASE_SEED + 31)
        q = torch.randn((B, Hq, D), generator=gen, device=dev).to(torch.bfloat16)
        kn = torch.randn((B, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
        vn = torch.randn((B, Hkv, D), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)
        ip = np.ascontiguousarray(batch.block_indptr, np.uint32)
        ids = np.ascontiguousarray(batch.block_ids, np.uint32)
        with DeviceKvPool(desc) as pool:
            plan = pool.plan(batch.ctx_lens, block_indptr=ip, block_ids=ids)
            info = plan.info()
            for _ in range(args.warmup):
                for layer in range(L):
                    pool.decode_step(layer, plan, kn, vn, q, None, None, out=out)
            torch.cuda.synchronize()
            n = max(args.steps, 1) * 5
            t0 = time.perf_counter()
            for _ in range(n):
                for layer in range(L):
                    pool.decode_step(layer, plan, kn, vn, q, None, None, out=out)
            torch.cuda.synchronize()
            us = (time.perf_counter() - t0) / (n * L) * 1e6
            pool.check()
            plan.close()
        kv = int(np.sum(batch.ctx_lens)) * desc.num_kv_heads * desc.head_dim * desc.elem_bytes * 2
        rows.append({"sequences": B, "context": ctxs[0], "plan": info, "us_per_layer": round(us, 2),
                     "kv_bytes_per_layer": kv, "kv_gbs": round(kv / us / 1e3, 1)})
    print(json.dumps({
        "metric": "latency-bound decode step: microseconds per layer", "unit": "us", "higher_is_better": False,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V from a seed in the pool (uninitialised blocks), q and new rows from a seed",
        "config": {"workload": "decode step (fused append + paged attention + merge) of 1-12 sequences, "
                               "Qwen2.5-7B heads", "layers_timed": 4, "q_heads": Hq, "kv_heads": Hkv,
                   "head_dim": D},
        "batches": rows}), flush=True)


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one MI355X and this path runs "
              f"on a single device (requested --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    if args.op == "prep":
        bench_prep(args)
        return
    if args.op == "wire":
        bench_wire(args)
        return
    if args.op in ("gather", "copy", "append"):
        bench_move(args)
        return
    if args.op == "extend":
        bench_extend(args)
        return
    if args.op == "shared":
        print(json.dumps(bench_shared(args.steps, args.warmup, cpu=not args.no_cpu_baseline,
                                      cpu_seconds=args.cpu_seconds)), flush=True)
        return
    if args.op == "pressure":
        print(json.dumps(bench_pressure(args.steps, args.warmup, cpu=not args.no_cpu_baseline,
                                        cpu_seconds=args.cpu_seconds)), flush=True)
        return
    if args.op == "small":
        bench_small(args)
        return
    from mitten_amd import workloads as wl

    kernel = None if args.kernel == "auto" else args.kernel
    result, batch, step_bytes = decode_config(args.config, args.steps, args.warmup, args.mode, args.pieces, kernel,
                                              args.split_tokens, not args.no_launch_events)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl.CONFIGS[args.config], batch, step_bytes, args.cpu_seconds)
    if args.configs and args.config == "qwen2.5-7b" and args.mode == "step":
        # The other configurations of the measurement table, each on its own
        # pool at its full size, with fewer steps (their own lines come from
        # --config / --op).
        ks, kw = max(4, min(args.steps, 12)), max(1, min(args.warmup, 2))
        cpu = not args.no_cpu_baseline
        nested = {}
        for name in ("qwen2.5-0.5b", "gemma-2b-mqa"):
            r, b, sb = decode_config(name, ks, kw)
            if cpu:
                r["cpu_baseline"] = cpu_baseline(wl.CONFIGS[name], b, sb, args.cpu_seconds, paged=False)
            nested[name] = _nested(r)
        nested["radix-shared-prefix"] = _nested(bench_shared(ks, kw, cpu=cpu, compare_whole=False,
                                                             cpu_seconds=args.cpu_seconds))
        nested["pool-pressure"] = _nested(bench_pressure(ks, kw, cpu=cpu, cpu_seconds=args.cpu_seconds))
        result["configs"] = nested
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
