"""Decode-step benchmark of the paged-KV hot path on one MI355X.

One step = for every layer of the Qwen2.5-7B-shaped batch (28 layers, 28 query
heads, 4 KV heads, head_dim 128, bf16 KV, block size 16, 64 sequences with
context lengths uniform in [1024, 8192], block tables drawn from a seeded
permutation of the pool): append the step's K/V row of every sequence into its
slot, then run paged GQA decode attention over context + 1 tokens.

Prints one JSON line: whole-step HBM throughput in algorithmic bytes (K/V
read once, Q read, O written, appends read+written, block tables and slot
ids), tokens/s, the attention kernel's roofline fraction measured with HIP
events on its stream over the timed region, and the CPU baseline (the
oracle's reference-faithful restatement of the reference's CPU attention,
timed on a bounded sample on this host).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

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
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
METRIC = "paged KV append+decode-attn achieved HBM GB/s (% peak); decode tokens/s"


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
    ap.add_argument("--no-launch-events", action="store_true",
                    help="time the steps without per-launch HIP events (roofline fields null)")
    ap.add_argument("--cpu-layers", type=int, default=5,
                    help="layers of the batch in the CPU baseline sample")
    ap.add_argument("--op", choices=["decode", "prep", "wire", "gather", "copy", "extend", "shared", "pressure"],
                    default="decode",
                    help="decode: the decode step (headline); prep: the fused q/k-norm + RoPE + "
                         "append kernel on a prefill chunk; wire: KV block export + import of a "
                         "handoff; gather: block-table gather of the decode batch, one layer; "
                         "copy: copy_blocks of --copy-pairs block pairs, all layers; extend: chunked-"
                         "prefill attention of --extend-seqs chunks of --tokens-per-chunk after "
                         "--prefix tokens; shared: decode step of 256 sequences over a radix-shared "
                         "prefix, with its copy-on-write copies and compaction moves; pressure: "
                         "chunk appends + decode step over a 200 GB pool")
    ap.add_argument("--extend-seqs", type=int, default=8, help="--op extend: sequences")
    ap.add_argument("--tokens-per-chunk", type=int, default=512, help="--op extend: chunk length")
    ap.add_argument("--prefix", type=int, default=4096, help="--op extend: cached tokens before the chunk")
    ap.add_argument("--copy-pairs", type=int, default=4096, help="--op copy: block pairs")
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


def profiled_traffic(config: str, mode: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary of this
    workload (FETCH_SIZE and WRITE_SIZE, scaled by a 1 GiB copy kernel)."""
    path = os.path.join(ROOT, "profiles", f"decode_{mode}_{config}_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
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


def cpu_baseline(cfg, batch, step_bytes, layers, paged=True):
    """Reference-faithful CPU decode (contiguous f32 cache grown by a copy per
    token, repeat_kv materialised, mask, softmax, matmuls) for `layers` layers
    of every sequence of the batch, scaled to a full step. The primary figure
    is one thread, sequences one after another, as the reference executes
    requests serially (inference-backend/src/burn_backend.rs:44-71); one layer
    of the same sample threaded over sequences is reported beside it."""
    from oracle import oracle as orc

    ctx = batch.ctx_lens
    layers = max(1, min(layers, cfg["num_layers"]))
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    orc.set_num_threads(1)
    t1 = sum(orc.ref_faithful_batch(ctx, cfg["num_kv_heads"], cfg["num_q_heads"], cfg["head_dim"],
                                    seed=1 + layer) for layer in range(layers))
    orc.set_num_threads(threads)
    tn = orc.ref_faithful_batch(ctx, cfg["num_kv_heads"], cfg["num_q_heads"], cfg["head_dim"], seed=100)
    step_1t, step_nt = t1 / layers * cfg["num_layers"], tn * cfg["num_layers"]
    out = {
        "value": round(step_bytes / step_1t / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{layers} of {cfg['num_layers']} layers x all {batch.num_seqs} sequences, 1 thread, "
                   f"{t1:.1f} s; scaled to a full step"),
        "tokens_per_s": round(batch.num_seqs / step_1t, 2),
        "ms_per_step": round(step_1t * 1e3, 1),
        "threaded": {"value": round(step_bytes / step_nt / 1e9, 3), "unit": "GB/s", "cores": threads,
                     "tokens_per_s": round(batch.num_seqs / step_nt, 2),
                     "sample": f"1 layer of the sample, {threads} threads over sequences, {tn:.1f} s"},
        "cpu_model": cpu_info(),
        "host_cpus": os.cpu_count(),
    }
    if not paged:
        return out
    # Second line: the efficient paged oracle (f32 accumulation over a bf16 /
    # f32 pool, threaded over sequences and heads) on one layer of the same
    # batch, K/V from a seeded host pool of the same blocks; scaled to a step.
    es = 2 if cfg["dtype"] == "bf16" else 4
    od = orc.desc(1, cfg["num_kv_heads"], cfg["head_dim"], batch.num_blocks, es)
    raw = np.random.default_rng(7).standard_normal(orc.pool_bytes(od) // es, dtype=np.float32)
    host = orc.f32_to_bf16(raw) if es == 2 else raw
    del raw
    q = np.random.default_rng(8).standard_normal((batch.num_seqs, cfg["num_q_heads"], cfg["head_dim"]),
                                                 dtype=np.float32)
    c0 = time.perf_counter()
    orc.decode_attention(od, host, 0, q, batch.block_indptr, batch.block_ids, ctx)
    tp = time.perf_counter() - c0
    del host
    step_p = tp * cfg["num_layers"]
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
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        pool.check()
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
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
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
        else:
            rng = wl.SplitMix64(batch.seed + 5)
            perm = wl.permutation(batch.num_blocks, rng)
            npairs = args.copy_pairs
            src, dst = i32(perm[:npairs]), i32(perm[npairs:2 * npairs])
            launch_bytes = 2 * npairs * L * 2 * desc.block_bytes + 8 * npairs

            def launch(i):
                pool.copy_blocks(src, dst, stream=stream)
            kernel, what = "mkv_copy_blocks", f"{args.config} pool: {npairs} block pairs, all {L} layers, K and V"
        for i in range(args.warmup):
            launch(i)
        torch.cuda.synchronize()
        pool.check()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
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
            else:
                ps = min(64, npairs)
                orc.copy_blocks(od, host, perm[:ps], perm[npairs:npairs + ps])
                cpu_bytes = 2 * ps * L * 2 * desc.block_bytes
                sample = f"oracle copy_blocks of {ps} pairs, all layers"
            reps += 1
        cpu_s = (time.perf_counter() - c0) / reps
    launch_s = float(np.mean([a.elapsed_time(b) for a, b in evs])) / 1e3
    gbs = launch_bytes / launch_s / 1e9
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
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
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
    of the step, then per layer `pre_layer(layer)` (if given) and the fused
    append + attention."""
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

    def step():
        # The engine's per-step call: host page tables (u32 CSR) into the plan.
        plan.build(ctx_host, 0, stream=stream, block_indptr=ip, block_ids=ix)
        for layer in range(L):
            if pre_layer is not None:
                pre_layer(layer)
            run_layer(layer)

    return step


def _time_steps(step, steps, warmup, stream):
    """Wall-clock seconds per step over `steps` steps after `warmup`, and the
    HIP-event average of one step on `stream`."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for a_, b_ in evs:
        a_.record(stream)
        step()
        b_.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    ev = float(np.mean([a_.elapsed_time(b_) for a_, b_ in evs])) / 1e3
    return wall, ev


def _time_copies(pool, src, dst, reps, stream):
    """HIP-event average seconds of one copy_blocks launch of the pairs."""
    import torch

    dev = torch.device("cuda:0")
    s_, d_ = (torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev) for a in (src, dst))
    pool.copy_blocks(s_, d_, stream=stream)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a_, b_ in evs:
        a_.record(stream)
        pool.copy_blocks(s_, d_, stream=stream)
        b_.record(stream)
    torch.cuda.synchronize()
    pool.check()
    return float(np.mean([a_.elapsed_time(b_) for a_, b_ in evs])) / 1e3


def bench_shared(args):
    """Decode step over a radix-shared prefix (the prefix-sharing
    configuration): 256 sequences share a 4,100-token prefix after
    copy-on-write, so the prefix's 256 full blocks are the same ids in every
    table and each sequence owns its copy of the partial block and a suffix
    of ~U{64..1024} tokens. One step = the host plan, then fused append +
    attention for all 28 layers, as in the headline. GB/s is reported on
    unique bytes (every shared block counted once: the HBM figure) and on
    logical bytes (each sequence's whole context, what per-sequence caches
    would read). The value is mkv_decode_step_shared_prefix's step; the
    same step through mkv_decode_step over the whole tables (cached and
    non-temporal loads) is timed beside it. The copy-on-write copies (255 partial blocks) and a
    compaction's batched moves (a fifth of the blocks) are timed as
    copy_blocks launches over all layers, in GB/s of the moved bytes."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS["qwen2.5-7b"]
    L, Hq, Hkv, D = cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    seqs, prefix = 256, 4100
    batch = wl.shared_prefix_batch(seqs, prefix, 64, 1024, wl.SplitMix64(wl.BASE_SEED + 3))
    desc = PoolDesc(L, Hkv, Hq, D, batch.num_blocks, "bf16")
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    row = 2 * Hkv * D * 2  # K and V bytes of one token in one layer
    qo_meta = wl.algorithmic_bytes_attention(batch, Hq, Hkv, D, 2) - batch.total_tokens * row
    app = wl.algorithmic_bytes_append(seqs, Hkv, D, 2)
    logical = L * (batch.total_tokens * row + qo_meta + app)
    unique = L * (batch.meta["unique_tokens"] * row + qo_meta + app)
    with DeviceKvPool(desc) as pool:
        gen = torch.Generator(device=dev)
        gen.manual_seed(wl.BASE_SEED + 3)
        view = pool.tensor()
        for layer in range(L):
            view[layer].normal_(generator=gen)
        del view
        plan = pool.plan(batch.ctx_lens, stream=stream)
        # The tables share the prefix's blocks, so the loads go through the
        # caches (MKV_ATTN_CACHED_LOADS), as an engine would ask when its
        # radix cache hands out shared blocks; the non-temporal default is
        # timed beside it.
        step = _decode_step_run(pool, plan, batch, L, Hq, Hkv, D, wl.BASE_SEED + 33, dev, stream,
                                cached_loads=True)
        wall, ev = _time_steps(step, args.steps, args.warmup, stream)
        step_nt = _decode_step_run(pool, plan, batch, L, Hq, Hkv, D, wl.BASE_SEED + 33, dev, stream)
        wall_nt, _ = _time_steps(step_nt, args.steps, args.warmup, stream)
        pool.check()
        info = plan.info()
        plan.close()
        # The shared-prefix step (mkv_decode_step_shared_prefix): the prefix
        # read once for all 256 sequences on MFMA tiles, the suffixes through
        # a suffix plan, both merged.
        full = prefix // 16
        ip = batch.block_indptr
        sptr = (ip - full * np.arange(seqs + 1)).astype(np.int32)
        sids = np.concatenate([batch.block_ids[ip[b] + full:ip[b + 1]] for b in range(seqs)]).astype(np.int32)
        slen = (batch.ctx_lens - 16 * full).astype(np.int32)
        i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
        splan = pool.plan_suffixes(slen, stream=stream)
        gen2 = torch.Generator(device=dev)
        gen2.manual_seed(wl.BASE_SEED + 33)
        bf = lambda *shape: torch.randn(shape, generator=gen2, device=dev, dtype=torch.float32).to(torch.bfloat16)
        q, kn, vn = bf(L, seqs, Hq, D), bf(L, seqs, Hkv, D), bf(L, seqs, Hkv, D)
        out = torch.empty_like(q)
        run_sp = pool.bind_decode_step_shared_prefix(splan, kn, vn, q, i32(batch.meta["shared_blocks"]), i32(sptr),
                                                     i32(sids), out, stream=stream)

        def step_sp():
            splan.build(slen, 0, stream=stream)
            for layer in range(L):
                run_sp(layer)

        wall_sp, ev_sp = _time_steps(step_sp, args.steps, args.warmup, stream)
        pool.check()
        splan.close()
        # Copy-on-write: the last holder keeps the prefix's partial block, the
        # other 255 sequences get copies. Compaction: a fifth of the blocks
        # move from the top of the id space into holes below it.
        own = batch.meta["own_first"]
        cow_src, cow_dst = np.full(seqs - 1, own[0], np.int32), own[1:].astype(np.int32)
        n_mv = batch.num_blocks // 5
        mv_src = np.arange(batch.num_blocks - n_mv, batch.num_blocks, dtype=np.int32)
        mv_dst = wl.permutation(batch.num_blocks - n_mv, wl.SplitMix64(wl.BASE_SEED + 35))[:n_mv].astype(np.int32)
        per_pair = L * 2 * 16 * Hkv * D * 2 * 2 + 8
        cow_s = _time_copies(pool, cow_src, cow_dst, args.steps, stream)
        mv_s = _time_copies(pool, mv_src, mv_dst, args.steps, stream)
    result = {
        "metric": "shared-prefix decode step: HBM GB/s on unique bytes (% peak); effective GB/s on logical bytes",
        "value": round(unique / wall_sp / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall_sp * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V/Q from a seed; shared prefix ids and own blocks from a seeded permutation",
        "config": {"workload": f"radix-shared decode step: {seqs} sequences over one {prefix}-token prefix "
                               f"(suffixes U[64, 1024]), Qwen2.5-7B heads, {L} layers",
                   "layers": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block_size": 16,
                   "sequences": seqs, "prefix_tokens": prefix, "shared_blocks": int(batch.meta["shared_blocks"].size),
                   "tokens_attended": batch.total_tokens, "unique_tokens": batch.meta["unique_tokens"],
                   "pool_blocks": batch.num_blocks, "plan": info},
        "pct_peak": round(100.0 * unique / wall_sp / 1e9 / PEAK_HBM_GBS, 2),
        "effective_gbs_logical": round(logical / wall_sp / 1e9, 2),
        "logical_bytes_per_step": logical, "unique_bytes_per_step": unique,
        "tokens_per_s": round(seqs / wall_sp, 1),
        "step_us_hip_events": round(ev_sp * 1e6, 1),
        "entry": "mkv_decode_step_shared_prefix (prefix once on MFMA tiles, suffix plan, merge)",
        "whole_tables_cached_loads": {"entry": "mkv_decode_step, MKV_ATTN_CACHED_LOADS",
                                      "ms_per_step": round(wall * 1e3, 4), "step_us_hip_events": round(ev * 1e6, 1),
                                      "effective_gbs_logical": round(logical / wall / 1e9, 2),
                                      "unique_gbs": round(unique / wall / 1e9, 2)},
        "whole_tables_nontemporal": {"entry": "mkv_decode_step", "ms_per_step": round(wall_nt * 1e3, 4),
                                     "effective_gbs_logical": round(logical / wall_nt / 1e9, 2),
                                     "unique_gbs": round(unique / wall_nt / 1e9, 2)},
        "cow_copies": {"pairs": int(cow_src.size), "bytes": int(cow_src.size) * per_pair,
                       "avg_launch_us": round(cow_s * 1e6, 2),
                       "gbs": round(cow_src.size * per_pair / cow_s / 1e9, 2)},
        "compaction_moves": {"pairs": int(n_mv), "bytes": int(n_mv) * per_pair,
                             "avg_launch_us": round(mv_s * 1e6, 2),
                             "gbs": round(n_mv * per_pair / mv_s / 1e9, 2)},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, batch, logical, 1)
        result["cpu_baseline"]["bytes"] = "logical (each sequence's whole context)"
    print(json.dumps(result), flush=True)


def bench_pressure(args):
    """One step of a pool under pressure (the pool-pressure configuration):
    the 217,982-block pool of a 200 GB budget (all 28 layers, Qwen2.5-7B
    heads), 512 sequences with log-normal lengths (median 2,048, sigma 1,
    capped at 32,768) in blocks from a seeded permutation of the pool. Per
    step and layer, 8 sequences append a 512-token chunk (mkv_append) and
    the other 504 run the fused append + decode attention; the chunks'
    prefill attention is left out, as the configuration states."""
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS["qwen2.5-7b"]
    L, Hq, Hkv, D = cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    nblocks, seqs, chunk, chunk_seqs = 217_982, 512, 512, 8
    batch, chunk_slots, lengths = wl.pool_pressure_step(nblocks, seqs, chunk, chunk_seqs,
                                                        wl.SplitMix64(wl.BASE_SEED + 4))
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
        cs = torch.from_numpy(chunk_slots).to(dev)

        def chunk_append(layer):
            pool.append(layer, kc[layer], vc[layer], cs, stream=stream)

        plan = pool.plan(batch.ctx_lens, stream=stream)
        step = _decode_step_run(pool, plan, batch, L, Hq, Hkv, D, wl.BASE_SEED + 44, dev, stream,
                                pre_layer=chunk_append)
        wall, ev = _time_steps(step, args.steps, args.warmup, stream)
        pool.check()
        info = plan.info()
        plan.close()
        pool_bytes = pool.nbytes
    result = {
        "metric": "pool-pressure step (chunk appends + fused decode step): achieved HBM GB/s (% peak)",
        "value": round(step_bytes / wall / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,1) K/V/Q from a seed; log-normal lengths and block ids from a seeded permutation",
        "config": {"workload": f"pool-pressure step: {nblocks}-block pool ({pool_bytes / 1e9:.1f} GB), {seqs} "
                               f"log-normal sequences, {chunk_seqs} x {chunk}-token chunk appends + "
                               f"{batch.num_seqs} decodes, Qwen2.5-7B heads, {L} layers",
                   "layers": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block_size": 16,
                   "pool_blocks": nblocks, "pool_bytes": pool_bytes, "sequences": seqs,
                   "tokens_held": int(lengths.sum()), "decode_sequences": batch.num_seqs,
                   "tokens_attended": batch.total_tokens, "chunk_tokens": n_chunk, "plan": info},
        "pct_peak": round(100.0 * step_bytes / wall / 1e9 / PEAK_HBM_GBS, 2),
        "step_bytes": step_bytes, "tokens_per_s": round((batch.num_seqs + n_chunk) / wall, 1),
        "step_us_hip_events": round(ev * 1e6, 1),
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, batch, step_bytes, 1, paged=False)
    print(json.dumps(result), flush=True)


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
    if args.op in ("gather", "copy"):
        bench_move(args)
        return
    if args.op == "extend":
        bench_extend(args)
        return
    if args.op == "shared":
        bench_shared(args)
        return
    if args.op == "pressure":
        bench_pressure(args)
        return
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc
    from mitten_amd import workloads as wl

    cfg = wl.CONFIGS[args.config]
    batch = wl.config_batch(args.config)
    L, Hq, Hkv, D, dt = cfg["num_layers"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"], cfg["dtype"]
    B = batch.num_seqs
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
    kernel = None if args.kernel == "auto" else args.kernel
    ws = torch.empty(max(1, pool.workspace_size(B, max_ctx, args.split_tokens)), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    attn_bytes = wl.algorithmic_bytes_attention(batch, Hq, Hkv, D, es)
    app_bytes = wl.algorithmic_bytes_append(B, Hkv, D, es)
    step_bytes = L * (attn_bytes + app_bytes)
    # Bytes of the launch the HIP events bracket: the fused step moves the
    # append's bytes too.
    launch_bytes = attn_bytes + (app_bytes if args.mode == "step" else 0)

    ctx_host = batch.ctx_lens.copy()
    ip_h, ids_h = batch.block_indptr.astype(np.uint32), batch.block_ids.astype(np.uint32)
    plan = pool.plan(ctx_host, pieces=args.pieces, stream=stream, block_indptr=ip_h, block_ids=ids_h)

    run_layer = pool.bind_decode_step(plan, k_new, v_new, q, None, None, out, kernel=kernel, stream=stream)

    def step(events=None):
        """events: None, or L+1 timing events recorded between launches (the
        fused step has nothing else between consecutive layers)."""
        if args.mode != "split":
            # The engine's one call per step: host lengths and host page
            # tables (u32 CSR), validated, copied and uploaded with the plan.
            plan.build(ctx_host, args.pieces, stream=stream, block_indptr=ip_h, block_ids=ids_h)
        for layer in range(L):
            if args.mode != "step":
                pool.append(layer, k_new[layer], v_new[layer], slots, stream=stream)
            if events is not None:
                events[layer].record(stream)
            if args.mode == "step":
                run_layer(layer)
            elif args.mode == "planned":
                pool.decode_attention_planned(layer, plan, q[layer], None, None, out=out[layer],
                                              kernel=kernel, stream=stream)
            else:
                pool.decode_attention(layer, q[layer], indptr, ids, ctx, max_ctx, out=out[layer],
                                      split_tokens=args.split_tokens, workspace=ws, kernel=kernel,
                                      stream=stream)
        if events is not None:
            events[L].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    pool.check()

    # Launch timing: an event chain around every layer's launch on every
    # EVENT_EVERY-th timed step (events cost GPU time; sampling keeps the
    # timed steps close to unperturbed).
    EVENT_EVERY = 4
    timed = [s for s in range(args.steps) if s % EVENT_EVERY == 0 and not args.no_launch_events]
    ev = {s: [torch.cuda.Event(enable_timing=True) for _ in range(L + 1)] for s in timed}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(ev.get(s))
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    pool.check()
    elapsed = t1 - t0
    ms_step = elapsed / args.steps * 1e3
    attn_ms = [e[i].elapsed_time(e[i + 1]) for e in ev.values() for i in range(L)] or [float("nan")]
    attn_avg_s = float(np.mean(attn_ms)) / 1e3
    gbs = step_bytes / (elapsed / args.steps) / 1e9
    attn_gbs = launch_bytes / attn_avg_s / 1e9

    traffic, traffic_src = profiled_traffic(args.config, args.mode)
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic: N(0,1) K/V/Q from a seed; block tables from a seeded permutation of the pool",
        "config": {"workload": f"{args.config} decode step (append + paged decode attention per layer)",
                   "layers": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block_size": 16,
                   "sequences": B, "ctx_range": [cfg["ctx_lo"], cfg["ctx_hi"]],
                   "tokens_attended": batch.total_tokens, "pool_blocks": batch.num_blocks,
                   "pool_bytes": pool.nbytes, "seed": batch.seed, "mode": args.mode,
                   "plan": plan.info(), "split_tokens": args.split_tokens, "kernel": args.kernel},
        "pct_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "tokens_per_s": round(B / (elapsed / args.steps), 1),
        "step_bytes": step_bytes,
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": {"step": "mkv_decode_step (append + attention + merge, per layer)",
                                "planned": "mkv_decode_attention_planned (attention + merge, per layer)",
                                "split": "mkv_decode_attention (attention + merge, per layer)"}[args.mode],
                     "bytes_per_launch": launch_bytes, "avg_launch_us": round(attn_avg_s * 1e6, 2),
                     "launches_timed": len(attn_ms) if ev else 0},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, batch, step_bytes, args.cpu_layers)
    plan.close()
    pool.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
