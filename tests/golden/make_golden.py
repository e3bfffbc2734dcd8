"""Writes the golden fixtures in this directory from the CPU oracle.

Each .npz holds the inputs and expected outputs of one small case (numpy
arrays only; loaded with allow_pickle=False). Regenerate with
    python tests/golden/make_golden.py
and review the diff: the fixtures pin the oracle's current results.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402


def pool(seed, L, H, D, nblocks, es):
    d = orc.desc(L, H, D, nblocks, es)
    x = orc.fill_normal(seed, int(np.prod(orc.pool_shape(d)))).reshape(orc.pool_shape(d))
    return d, (x if es == 4 else orc.f32_to_bf16(x))


def rows(seed, shape, es):
    x = orc.fill_normal(seed, int(np.prod(shape))).reshape(shape)
    return x if es == 4 else orc.f32_to_bf16(x)


def main():
    out = {}
    # append: f32 and bf16, slots spread over blocks and offsets
    for name, es, D in (("append_f32", 4, 16), ("append_bf16", 2, 32)):
        d, p = pool(1, 2, 2, D, 4, es)
        slots = np.array([0, 17, 63, 5, 40, 33], np.int32)
        k, v = rows(2, (6, 2, D), es), rows(3, (6, 2, D), es)
        want = p.copy()
        assert orc.append(d, want, 1, k, v, slots) == -1
        out[name] = dict(pool=p, k=k, v=v, slots=slots, layer=np.int32(1), expected_pool=want,
                         geometry=np.array([2, 2, D, 4, es], np.int32))
    # gather (bf16): ragged contexts with partial last blocks
    d, p = pool(4, 1, 2, 32, 6, 2)
    indptr = np.array([0, 1, 3, 6], np.int32)
    ids = np.array([5, 0, 3, 2, 4, 1], np.int32)
    ctx = np.array([7, 32, 33], np.int32)
    gk, gv = orc.gather(d, p, 0, indptr, ids, ctx)
    out["gather_bf16"] = dict(pool=p, indptr=indptr, ids=ids, ctx=ctx, expected_k=gk, expected_v=gv,
                              geometry=np.array([1, 2, 32, 6, 2], np.int32))
    # copy_blocks (bf16): COW-style and compaction-style pairs, all layers
    d, p = pool(5, 3, 1, 16, 8, 2)
    src, dst = np.array([7, 6, 2], np.int32), np.array([0, 1, 4], np.int32)
    want = p.copy()
    orc.copy_blocks(d, want, src, dst)
    out["copy_blocks_bf16"] = dict(pool=p, src=src, dst=dst, expected_pool=want,
                                   geometry=np.array([3, 1, 16, 8, 2], np.int32))
    # decode attention: f32 GQA, bf16 GQA with the phantom zero key
    for name, es, Hq, Hkv, zs in (("attention_f32", 4, 4, 2, 0), ("attention_bf16_zero_sink", 2, 8, 2, 1)):
        d, p = pool(6, 1, Hkv, 32, 8, es)
        indptr = np.array([0, 1, 3, 7], np.int32)
        ids = np.array([6, 1, 4, 0, 2, 3, 5], np.int32)
        ctx = np.array([1, 17, 61], np.int32)
        q = rows(7, (3, Hq, 32), es)
        qf = q if es == 4 else orc.bf16_to_f32(q)
        o = orc.decode_attention(d, p, 0, qf, indptr, ids, ctx, zero_sink=bool(zs))
        out[name] = dict(pool=p, q=q, indptr=indptr, ids=ids, ctx=ctx, zero_sink=np.int32(zs),
                         expected_o=o, geometry=np.array([1, Hkv, 32, 8, es], np.int32),
                         q_heads=np.int32(Hq))
    for name, arrays in out.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
