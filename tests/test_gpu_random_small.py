"""Seeded random decode steps small enough to take the per-sequence kernel:
the per-head (VALU) path (f32 pools, or bf16 with kernel "valu") on fewer
(block, KV head) units than two per CU, where one workgroup per (sequence, KV
head, query head) merges its waves' states in LDS and no merge launch
follows. Random head shapes, 1-8 sequences, contexts from one token to the
size limit, piece counts, the zero sink, host or device tables, and the
fused block-table gather (the engine's small-model step,
inference-model-qwen/src/model.rs:390-416 with the contiguous per-sequence
K/V of :391-392). Pool, gather and attention are checked against the
oracle."""
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
    (12, 2, 32, "f32", None),
    (8, 1, 256, "f32", None),
    (28, 4, 128, "f32", None),
    (7, 1, 128, "f32", None),
    (16, 16, 64, "f32", None),
    (14, 2, 64, "bf16", "valu"),
    (28, 4, 128, "bf16", "valu"),
    (8, 1, 256, "bf16", "valu"),
    (32, 8, 32, "bf16", "valu"),
]

N_CASES = 24
UNITS = 480  # (block, KV head) units per launch: below two per CU of the MI355X's 256


def _case(i: int):
    rng = np.random.default_rng(12000 + i)
    Hq, Hkv, D, dt, kernel = KINDS[int(rng.integers(len(KINDS)))]
    B = int(rng.integers(1, 9))
    per_seq = max(1, UNITS // (Hkv * B))  # blocks per sequence at most
    ctx = [int(rng.integers(1, 16 * per_seq + 1)) for _ in range(B)]
    total = sum((c + 15) // 16 for c in ctx)
    pieces = [0, 1, int(rng.integers(1, total + 6))][int(rng.integers(3))]
    return dict(Hq=Hq, Hkv=Hkv, D=D, dt=dt, kernel=kernel, ctx=ctx, pieces=pieces,
                zero_sink=bool(rng.integers(2)), host_tables=bool(rng.integers(2)), gather=bool(rng.integers(2)),
                seed=12100 + 10 * i)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_small_step_matches_the_oracle(i):
    import torch

    c = _case(i)
    B = len(c["ctx"])
    print(f"case {i}: Hq {c['Hq']} Hkv {c['Hkv']} D {c['D']} {c['dt']} kernel {c['kernel']} B {B} ctx {c['ctx']} "
          f"pieces {c['pieces']} zero_sink {c['zero_sink']} host tables {c['host_tables']} gather {c['gather']}",
          flush=True)
    seed, dt, Hkv, D = c["seed"], c["dt"], c["Hkv"], c["D"]
    batch = wl.decode_batch_from_contexts([x - 1 for x in c["ctx"]], wl.SplitMix64(seed), extra_blocks=2)
    desc = PoolDesc(1, Hkv, c["Hq"], D, batch.num_blocks, dt)
    host = normal(seed + 1, desc.shape, dt)
    q = normal(seed + 2, (B, c["Hq"], D), dt)
    kn = normal(seed + 3, (B, Hkv, D), dt)
    vn = normal(seed + 4, (B, Hkv, D), dt)
    ip = np.ascontiguousarray(batch.block_indptr, np.uint32)
    ids = np.ascontiguousarray(batch.block_ids, np.uint32)
    ntok = int(sum(c["ctx"])) * Hkv * D
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        if c["host_tables"]:
            plan = pool.plan(batch.ctx_lens, pieces=c["pieces"], block_indptr=ip, block_ids=ids)
            tables = (None, None)
        else:
            plan = pool.plan(batch.ctx_lens, pieces=c["pieces"])
            tables = tuple(torch.from_numpy(a.astype(np.int32)).cuda() for a in (ip, ids))
        gout = None
        if c["gather"]:
            gk = torch.full((ntok + 8,), 7.0, dtype=pool.torch_dtype, device="cuda")
            gout = (gk, torch.full_like(gk, 7.0))
        o = pool.decode_step(0, plan, to_device(kn), to_device(vn), to_device(q), *tables,
                             zero_sink=c["zero_sink"], kernel=c["kernel"], gather_out=gout)
        pool.check()
        got, after = to_host(o), pool.read()
        if gout is not None:
            gk_h, gv_h = to_host(gout[0]), to_host(gout[1])
        plan.close()
    want = host.copy()
    assert orc.append(odesc(desc), want, 0, kn, vn, batch.slot_mapping) == -1
    assert np.array_equal(bits(after), bits(want)), "fused append is not bit-exact"
    if gout is not None:
        rk, rv = orc.gather(odesc(desc), want, 0, batch.block_indptr, batch.block_ids, batch.ctx_lens)
        assert np.array_equal(bits(gk_h[:ntok]), bits(rk)) and np.array_equal(bits(gv_h[:ntok]), bits(rv))
        assert np.all(widen(gk_h[ntok:]) == 7.0) and np.all(widen(gv_h[ntok:]) == 7.0), "gather wrote past its rows"
    ref = orc.decode_attention(odesc(desc), want, 0, widen(q), batch.block_indptr, batch.block_ids, batch.ctx_lens,
                               zero_sink=c["zero_sink"])
    assert_attention_close(got, ref, dt)
