"""Golden fixtures (tests/golden/*.npz, written by make_golden.py from the
oracle): the oracle must still reproduce them exactly (CPU), and the HIP
library must match them bit-exactly for KV movement and within tolerance for
attention (GPU)."""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import assert_attention_close, bits, to_device, to_host, widen

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "*.npz")))


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _desc(f):
    L, H, D, nb, es = (int(x) for x in f["geometry"])
    return orc.desc(L, H, D, nb, es)


def test_fixture_set_is_complete():
    assert set(FIXTURES) == {"append_f32", "append_bf16", "gather_bf16", "copy_blocks_bf16", "attention_f32",
                             "attention_bf16_zero_sink"}


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_fixture(name):
    f = load(name)
    d = _desc(f)
    if name.startswith("append"):
        p = f["pool"].copy()
        assert orc.append(d, p, int(f["layer"]), f["k"], f["v"], f["slots"]) == -1
        assert np.array_equal(bits(p), bits(f["expected_pool"]))
    elif name.startswith("gather"):
        k, v = orc.gather(d, f["pool"], 0, f["indptr"], f["ids"], f["ctx"])
        assert np.array_equal(bits(k), bits(f["expected_k"])) and np.array_equal(bits(v), bits(f["expected_v"]))
    elif name.startswith("copy"):
        p = f["pool"].copy()
        orc.copy_blocks(d, p, f["src"], f["dst"])
        assert np.array_equal(bits(p), bits(f["expected_pool"]))
    else:
        o = orc.decode_attention(d, f["pool"], 0, widen(f["q"]), f["indptr"], f["ids"], f["ctx"],
                                 zero_sink=bool(f["zero_sink"]))
        assert np.array_equal(o, f["expected_o"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_hip_library_matches_fixture(name):
    import torch

    from mitten_amd import DeviceKvPool, PoolDesc

    f = load(name)
    L, H, D, nb, es = (int(x) for x in f["geometry"])
    dt = "f32" if es == 4 else "bf16"
    Hq = int(f["q_heads"]) if "q_heads" in f else H
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()
    with DeviceKvPool(PoolDesc(L, H, Hq, D, nb, dt)) as pool:
        pool.write(f["pool"])
        if name.startswith("append"):
            pool.append(int(f["layer"]), to_device(f["k"]), to_device(f["v"]), i32(f["slots"]))
            pool.check()
            assert np.array_equal(bits(pool.read()), bits(f["expected_pool"]))
        elif name.startswith("gather"):
            ci = np.concatenate([[0], np.cumsum(f["ctx"])]).astype(np.int32)
            k, v = pool.gather(0, i32(f["indptr"]), i32(f["ids"]), i32(ci), int(f["ctx"].max()),
                               total_tokens=int(ci[-1]))
            pool.check()
            assert np.array_equal(bits(to_host(k)), bits(f["expected_k"]))
            assert np.array_equal(bits(to_host(v)), bits(f["expected_v"]))
        elif name.startswith("copy"):
            pool.copy_blocks(i32(f["src"]), i32(f["dst"]))
            pool.check()
            assert np.array_equal(bits(pool.read()), bits(f["expected_pool"]))
        else:
            zs = bool(f["zero_sink"])
            o = pool.decode_attention(0, to_device(f["q"]), i32(f["indptr"]), i32(f["ids"]), i32(f["ctx"]),
                                      int(f["ctx"].max()), zero_sink=zs)
            plan = pool.plan(f["ctx"], pieces=2)
            o2 = pool.decode_attention_planned(0, plan, to_device(f["q"]), i32(f["indptr"]), i32(f["ids"]),
                                               zero_sink=zs)
            pool.check()
            assert_attention_close(to_host(o), f["expected_o"], dt)
            assert_attention_close(to_host(o2), f["expected_o"], dt)
            plan.close()
