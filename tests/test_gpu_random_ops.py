"""Seeded random sequences of the pool's data-movement operations, each
checked bit for bit against the oracle on the same host copy of the pool:
append (one layer and all layers), the block-table gather, batched block
copies, and the wire export / import. Shapes (layers, KV heads, head_dim,
dtype, pool size), slot sets, tables, copy pairs and wire block lists are
drawn per case, in device-metadata and host-metadata forms. The pool starts
from random bytes (NaN patterns included), so every untouched slot is checked
too. Head dims include ones no attention kernel takes (8, 40, 96, 512): the
data-movement kernels work in 16-byte chunks of any row. The operations
follow inference-backend/src/kv_pool.rs (slots, blocks),
inference-model-qwen/src/model.rs:390-408 (append, contiguous per-sequence
K/V) and radix_cache.rs:243-282 (block moves)."""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import DeviceKvPool, PoolDesc
from oracle import oracle as orc
from tests.helpers import bits, normal, odesc, to_device, to_host

pytestmark = pytest.mark.gpu

N_CASES = 24
HEAD_DIMS = (8, 32, 40, 64, 96, 128, 256, 512)  # any multiple of 8 the pool accepts


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _case(i: int):
    rng = np.random.default_rng(11000 + i)
    dt = "f32" if rng.random() < 0.3 else "bf16"
    Hkv = int(rng.choice([1, 2, 4, 8]))
    return dict(rng=rng, L=int(rng.integers(1, 5)), Hkv=Hkv, Hq=Hkv * int(rng.integers(1, 8)),
                D=int(rng.choice(HEAD_DIMS)), nb=int(rng.integers(8, 161)), dt=dt, host=bool(rng.integers(2)),
                seed=11500 + 10 * i)


def _random_bits(desc: PoolDesc, seed: int) -> np.ndarray:
    raw = np.random.default_rng(seed).integers(0, 256, int(np.prod(desc.shape)) * desc.elem_bytes, dtype=np.uint8)
    return raw.view(np.float32 if desc.dtype == "f32" else np.uint16).reshape(desc.shape)


def _tables(rng: np.random.Generator, nb: int):
    """Random CSR block tables (ids may repeat across sequences, as shared
    prefix pages do) and context lengths that fit them."""
    B = int(rng.integers(1, 9))
    ctx = []
    ids = []
    indptr = [0]
    for _ in range(B):
        c = int(rng.integers(1, 16 * min(nb, 24) + 1))
        n = (c + 15) // 16 + int(rng.integers(0, 2))  # a table may hold one block past the context
        ids.extend(int(x) for x in rng.integers(0, nb, n))
        indptr.append(len(ids))
        ctx.append(c)
    return np.array(indptr, np.int32), np.array(ids, np.int32), np.array(ctx, np.int32)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_data_movement_matches_the_oracle(i):
    c = _case(i)
    rng, dt, host = c["rng"], c["dt"], c["host"]
    desc = PoolDesc(c["L"], c["Hkv"], c["Hq"], c["D"], c["nb"], dt)
    od = odesc(desc)
    print(f"case {i}: L {c['L']} Hkv {c['Hkv']} D {c['D']} {dt} blocks {c['nb']} host {host}", flush=True)
    ref = _random_bits(desc, c["seed"])
    slots_total = desc.num_blocks * desc.page_size
    with DeviceKvPool(desc) as pool:
        pool.write(ref)

        # One layer's append: unique slots anywhere in the pool.
        layer = int(rng.integers(c["L"]))
        n = int(rng.integers(1, min(300, slots_total) + 1))
        slots = rng.choice(slots_total, n, replace=False).astype(np.int32)
        k = normal(c["seed"] + 1, (n, c["Hkv"], c["D"]), dt)
        v = normal(c["seed"] + 2, (n, c["Hkv"], c["D"]), dt)
        pool.append(layer, to_device(k), to_device(v), slots.astype(np.uint32) if host else _i32(slots))
        assert orc.append(od, ref, layer, k, v, slots) == -1
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(ref)), "append"

        # Every layer at once.
        n2 = int(rng.integers(1, min(64, slots_total) + 1))
        slots2 = rng.choice(slots_total, n2, replace=False).astype(np.int32)
        ka = normal(c["seed"] + 3, (c["L"], n2, c["Hkv"], c["D"]), dt)
        va = normal(c["seed"] + 4, (c["L"], n2, c["Hkv"], c["D"]), dt)
        pool.append_all_layers(to_device(ka), to_device(va), slots2.astype(np.uint32) if host else _i32(slots2))
        for layer2 in range(c["L"]):
            assert orc.append(od, ref, layer2, ka[layer2], va[layer2], slots2) == -1
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(ref)), "append_all_layers"

        # Gather of random tables.
        indptr, ids, ctx = _tables(rng, c["nb"])
        layer = int(rng.integers(c["L"]))
        if host:
            gk, gv = pool.gather_host(layer, indptr.astype(np.uint32), ids.astype(np.uint32), ctx)
        else:
            ctx_indptr = np.concatenate([[0], np.cumsum(ctx)]).astype(np.int32)
            gk, gv = pool.gather(layer, _i32(indptr), _i32(ids), _i32(ctx_indptr), int(ctx.max()))
        pool.check()
        rk, rv = orc.gather(od, ref, layer, indptr, ids, ctx)
        total = int(ctx.sum()) * c["Hkv"] * c["D"]
        assert np.array_equal(bits(to_host(gk)[:total]), bits(rk)), "gather k"
        assert np.array_equal(bits(to_host(gv)[:total]), bits(rv)), "gather v"

        # Block copies: disjoint source and destination sets.
        npairs = int(rng.integers(1, c["nb"] // 2 + 1))
        perm = rng.permutation(c["nb"]).astype(np.int32)
        src, dst = perm[:npairs], perm[npairs:2 * npairs]
        if host:
            pool.copy_blocks(src.astype(np.uint32), dst.astype(np.uint32))
        else:
            pool.copy_blocks(_i32(src), _i32(dst))
        orc.copy_blocks(od, ref, src, dst)
        pool.check()
        assert np.array_equal(bits(pool.read()), bits(ref)), "copy_blocks"

        # Wire export of a random block list (repeats allowed) and layer range,
        # then import of the payload into distinct blocks.
        nw = int(rng.integers(1, min(40, c["nb"]) + 1))
        wids = rng.integers(0, c["nb"], nw).astype(np.int32)
        lb = int(rng.integers(c["L"]))
        nl = int(rng.integers(1, c["L"] - lb + 1))
        payload, sums = pool.wire_export(wids.astype(np.uint32) if host else _i32(wids), lb, nl)
        pool.check()
        ref_p, ref_s = orc.wire_export(od, ref, wids, lb, nl)
        assert np.array_equal(to_host(payload), ref_p), "wire payload"
        assert np.array_equal(to_host(sums), ref_s), "wire checksums"
        dids = rng.choice(c["nb"], nw, replace=False).astype(np.int32)
        got_s = pool.wire_import(dids.astype(np.uint32) if host else _i32(dids), payload, lb, nl, expected=sums)
        pool.check()
        assert np.array_equal(orc.wire_import(od, ref, dids, lb, nl, ref_p), ref_s)
        assert np.array_equal(to_host(got_s), ref_s), "wire import checksums"
        assert np.array_equal(bits(pool.read()), bits(ref)), "wire import"
