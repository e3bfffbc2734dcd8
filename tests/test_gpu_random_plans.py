"""Seeded random decode steps through the plan: random head shapes and
kernels, batch sizes, context lengths (block edges and single tokens
included), piece counts (0 = the device's choice, one piece, more pieces
than blocks), the zero sink, host or device page tables, and K/V loads
through the caches or not (MKV_ATTN_CACHED_LOADS). Each case runs
the fused append + attention step (`mkv_decode_step`) on one layer and checks
the pool bit for bit and the attention output against the oracle, as the
engine's decode step (inference-model-qwen/src/model.rs:390-416) computes
it."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import DeviceKvPool, PoolDesc
from mitten_amd import workloads as wl
from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

# (Hq, Hkv, D, dtype, kernel)
KINDS = [
    (14, 2, 64, "f32", None),
    (28, 4, 128, "bf16", "mfma"),
    (28, 4, 128, "bf16", "mfma-per-head"),
    (28, 4, 128, "bf16", "valu"),
    (8, 1, 256, "bf16", "mfma"),
    (14, 2, 64, "bf16", "mfma"),
    (32, 8, 128, "bf16", "mfma"),
    (64, 4, 128, "bf16", "mfma"),
    (16, 4, 256, "bf16", "mfma"),
    (12, 2, 32, "f32", None),
    (8, 1, 256, "f32", None),
]

N_CASES = 40


def _contexts(rng: np.random.Generator, B: int) -> list[int]:
    out = []
    for _ in range(B):
        r = rng.random()
        if r < 0.3:
            out.append(int(rng.integers(1, 41)))
        elif r < 0.6:
            out.append(max(1, 16 * int(rng.integers(1, 40)) + int(rng.integers(-1, 2))))
        else:
            out.append(int(rng.integers(1, 1501)))
    return out


def _case(i: int):
    rng = np.random.default_rng(9000 + i)
    Hq, Hkv, D, dt, kernel = KINDS[int(rng.integers(len(KINDS)))]
    B = int(rng.integers(1, 49))
    ctx = _contexts(rng, B)
    total = sum((c + 15) // 16 for c in ctx)
    pieces = [0, 1, int(rng.integers(1, total + 6))][int(rng.integers(3))]
    zero_sink, host_tables = bool(rng.integers(2)), bool(rng.integers(2))
    return dict(Hq=Hq, Hkv=Hkv, D=D, dt=dt, kernel=kernel, ctx=ctx, pieces=pieces, zero_sink=zero_sink,
                host_tables=host_tables, cached=bool(rng.integers(2)), seed=9100 + 10 * i)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_decode_step_matches_the_oracle(i):
    c = _case(i)
    print(f"case {i}: Hq {c['Hq']} Hkv {c['Hkv']} D {c['D']} {c['dt']} kernel {c['kernel']} B {len(c['ctx'])} "
          f"pieces {c['pieces']} zero_sink {c['zero_sink']} host tables {c['host_tables']} cached {c['cached']}",
          flush=True)
    seed, dt = c["seed"], c["dt"]
    batch = wl.decode_batch_from_contexts([x - 1 for x in c["ctx"]], wl.SplitMix64(seed), extra_blocks=2)
    desc = PoolDesc(1, c["Hkv"], c["Hq"], c["D"], batch.num_blocks, dt)
    B = len(c["ctx"])
    host = normal(seed + 1, desc.shape, dt)
    q = normal(seed + 2, (B, c["Hq"], c["D"]), dt)
    kn = normal(seed + 3, (B, c["Hkv"], c["D"]), dt)
    vn = normal(seed + 4, (B, c["Hkv"], c["D"]), dt)
    ip = np.ascontiguousarray(batch.block_indptr, np.uint32)
    ids = np.ascontiguousarray(batch.block_ids, np.uint32)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        if c["host_tables"]:
            plan = pool.plan(batch.ctx_lens, pieces=c["pieces"], block_indptr=ip, block_ids=ids)
            tables = (None, None)
        else:
            import torch

            plan = pool.plan(batch.ctx_lens, pieces=c["pieces"])
            tables = tuple(torch.from_numpy(a.astype(np.int32)).cuda() for a in (ip, ids))
        o = pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), *tables,
                             zero_sink=c["zero_sink"], kernel=c["kernel"], cached_loads=c["cached"])
        pool.check()
        got, after = to_host(o), pool.read()
        plan.close()
    want = host.copy()
    assert orc.append(odesc(desc), want, 0, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(after), bits(want)), "fused append is not bit-exact"
    ref = orc.decode_attention(odesc(desc), want, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens,
                               zero_sink=c["zero_sink"])
    assert_attention_close(got, ref, dt)
