"""Seeded random fused pre-attention steps (mkv_qk_norm_rope_append and its
host-metadata form): random head shapes (head_dim 32-256, 1-8 query heads per
KV head), rotary widths (none, any multiple the step accepts, the whole
head), RoPE bases, gated or plain q, with or without the norm, 1-600 tokens at
random or consecutive positions up to 65,535, random slots, either layer.
Checked against the oracle with the bars of test_gpu_prep.py: v rows and
every row the step does not write bit-exact, prepared q and k within the
f32 / bf16 tolerance (inference-model-qwen/src/model.rs:371-392, norm
:98-108, RoPE :508-540)."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import DeviceKvPool, PoolDesc
from mitten_amd.device_pool import rope_inv_freq
from oracle import oracle as orc
from tests.helpers import odesc, to_device, to_host, widen
from tests.test_gpu_prep import _close, _f32, _i32

pytestmark = pytest.mark.gpu

N_CASES = 24


def _case(i: int):
    rng = np.random.default_rng(13000 + i)
    D = int(rng.choice([32, 64, 128, 256]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    Hq = Hkv * int(rng.integers(1, 9))
    m = 2 * max(1, D // 64)  # rotary_dim granularity the step accepts
    r = rng.random()
    rd = 0 if r < 0.15 else D if r < 0.3 else m * int(rng.integers(1, D // m + 1))
    n = int(rng.integers(1, 601))
    return dict(Hq=Hq, Hkv=Hkv, D=D, rd=rd, theta=float(rng.choice([1e4, 1e6, 1e7])),
                dt="f32" if rng.random() < 0.3 else "bf16", gated=bool(rng.integers(2)), norm=bool(rng.integers(2)),
                n=n, consecutive=bool(rng.integers(2)), host=bool(rng.integers(2)), layer=int(rng.integers(2)),
                seed=13500 + 10 * i)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_prep_matches_the_oracle(i):
    c = _case(i)
    Hq, Hkv, D, rd, dt, n = c["Hq"], c["Hkv"], c["D"], c["rd"], c["dt"], c["n"]
    print(f"case {i}: Hq {Hq} Hkv {Hkv} D {D} rotary {rd} theta {c['theta']:g} {dt} gated {c['gated']} "
          f"norm {c['norm']} tokens {n} consecutive {c['consecutive']} host {c['host']} layer {c['layer']}",
          flush=True)
    rng = np.random.default_rng(c["seed"])
    nb = max(8, (n + 15) // 16 * 2)
    desc = PoolDesc(2, Hkv, Hq, D, nb, dt)
    base = rng.standard_normal(desc.shape).astype(np.float32)
    host = base if dt == "f32" else orc.f32_to_bf16(base)
    q = (rng.standard_normal((n, Hq, 2, D) if c["gated"] else (n, Hq, D)) * 2).astype(np.float32)
    k = (rng.standard_normal((n, Hkv, D)) * 2).astype(np.float32)
    v = rng.standard_normal((n, Hkv, D)).astype(np.float32)
    if dt == "bf16":
        q, k, v = (orc.f32_to_bf16(a) for a in (q, k, v))
    wq = rng.uniform(-0.5, 0.5, D).astype(np.float32) if c["norm"] else None
    wk = rng.uniform(-0.5, 0.5, D).astype(np.float32) if c["norm"] else None
    f = rope_inv_freq(rd, c["theta"]) if rd else None
    slots = rng.permutation(nb * 16)[:n].astype(np.int32)
    if c["consecutive"]:
        positions = (int(rng.integers(0, 65536 - n)) + np.arange(n)).astype(np.int32)
    else:
        positions = rng.integers(0, 65536, n).astype(np.int32)
    layer = c["layer"]
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        if c["host"]:
            meta = (positions, slots.astype(np.uint32))
        else:
            meta = (_i32(positions), _i32(slots))
        qo = pool.qk_norm_rope_append(layer, to_device(q), to_device(k), to_device(v), *meta,
                                      None if wq is None else _f32(wq), None if wk is None else _f32(wk),
                                      None if f is None else _f32(f), eps=1e-6, gated=c["gated"])
        pool.check()
        got_q, got_pool = to_host(qo), pool.read()
    ref_pool = host.copy()
    ref_q = orc.qk_norm_rope_append(odesc(desc), ref_pool, layer, widen(q), widen(k), widen(v), wq, wk, f, 1e-6,
                                    positions, slots)
    _close(got_q, ref_q, dt, "q")
    blk, off = slots // 16, slots % 16
    assert np.array_equal(got_pool[layer, 1, blk, off], ref_pool[layer, 1, blk, off]), "v rows"
    _close(got_pool[layer, 0, blk, off], ref_pool[layer, 0, blk, off], dt, "k rows")
    mask = np.ones(got_pool.shape[:4], bool)
    mask[layer, 0, blk, off] = False
    mask[layer, 1, blk, off] = False
    assert np.array_equal(got_pool[mask], ref_pool[mask]), "rows the step does not write"
