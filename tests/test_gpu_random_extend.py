"""Seeded random extend (chunked-prefill) attention: random head shapes (the
MFMA query tiles and the per-token segment path), batch sizes, cached
prefixes, chunk lengths (single tokens, whole prompts, chunks after a prefix,
and sequences with no new token), the zero sink, and the device or host
metadata form. Each case checks the causal attention of every new token over
its sequence's whole cache (inference-model-qwen/src/model.rs:410-416, mask
:542-555) against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import DeviceKvPool, PoolDesc
from mitten_amd import workloads as wl
from oracle import oracle as orc
from tests.helpers import assert_attention_close, normal, odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

# (Hq, Hkv, D, dtype)
KINDS = [
    (28, 4, 128, "bf16"),
    (8, 1, 256, "bf16"),
    (14, 2, 64, "bf16"),
    (32, 8, 128, "bf16"),
    (64, 4, 128, "bf16"),
    (4, 4, 64, "bf16"),
    (16, 4, 256, "bf16"),
    (16, 1, 256, "bf16"),
    (14, 2, 64, "f32"),
    (64, 2, 128, "bf16"),  # 32 query heads per KV head: per-token segments
    (8, 2, 32, "bf16"),    # head_dim 32: per-token segments
]

N_CASES = 24


def _case(i: int):
    rng = np.random.default_rng(7000 + i)
    Hq, Hkv, D, dt = KINDS[int(rng.integers(len(KINDS)))]
    B = int(rng.integers(1, 9))
    ctx, nq = [], []
    for _ in range(B):
        c = int(rng.integers(1, 1001))
        r = rng.random()
        n = 1 if r < 0.25 else min(c, 256) if r < 0.5 else 0 if r < 0.6 else int(rng.integers(1, min(c, 256) + 1))
        ctx.append(c)
        nq.append(n)
    if sum(nq) == 0:
        nq[0] = 1
    return dict(Hq=Hq, Hkv=Hkv, D=D, dt=dt, ctx=ctx, nq=nq, zero_sink=bool(rng.integers(2)),
                host=bool(rng.integers(2)), seed=7100 + 10 * i)


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_extend_matches_the_oracle(i):
    c = _case(i)
    print(f"case {i}: Hq {c['Hq']} Hkv {c['Hkv']} D {c['D']} {c['dt']} ctx {c['ctx']} new {c['nq']} "
          f"zero_sink {c['zero_sink']} host {c['host']}", flush=True)
    seed, dt = c["seed"], c["dt"]
    batch = wl.decode_batch_from_contexts([x - 1 for x in c["ctx"]], wl.SplitMix64(seed), extra_blocks=2)
    desc = PoolDesc(1, c["Hkv"], c["Hq"], c["D"], batch.num_blocks, dt)
    host = normal(seed + 1, desc.shape, dt)
    q_indptr = np.concatenate([[0], np.cumsum(c["nq"])]).astype(np.int32)
    q = normal(seed + 2, (int(q_indptr[-1]), c["Hq"], c["D"]), dt)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        if c["host"]:
            o = pool.extend_attention_host(0, to_device(q), c["nq"], batch.ctx_lens,
                                           np.ascontiguousarray(batch.block_indptr, np.uint32),
                                           np.ascontiguousarray(batch.block_ids, np.uint32),
                                           zero_sink=c["zero_sink"])
        else:
            o = pool.extend_attention(0, to_device(q), _i32(q_indptr), _i32(batch.block_indptr),
                                      _i32(batch.block_ids), _i32(batch.ctx_lens), max(c["nq"]), max(c["ctx"]),
                                      zero_sink=c["zero_sink"])
        pool.check()
        got = to_host(o)
    ref = orc.extend_attention(odesc(desc), host, 0, widen(q), q_indptr, batch.block_indptr, batch.block_ids,
                               batch.ctx_lens, zero_sink=c["zero_sink"])
    assert_attention_close(got, ref, dt)
