"""GPU parity of the fused pre-attention step (mkv_qk_norm_rope_append)
against the oracle: q/k RMSNorm(1 + w) + partial NeoX RoPE, k and v appended
at their slots, prepared q written out.

Bars: v rows and every untouched pool row bit-exact; f32 outputs within
1e-5 absolute; bf16 outputs within one bf16 ulp of the oracle's rounding of
its f32 result, plus 1e-5 of the head row's largest value (the f32 values
differ by a few f32 ulps of the operands: another summation order, another
sin/cos), with at least 99% of elements bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd import BackendError, DeviceIndexError, DeviceKvPool, PoolDesc
from mitten_amd import device_pool as dp
from mitten_amd.device_pool import rope_inv_freq
from oracle import oracle as orc
from tests.helpers import odesc, to_device, to_host, widen

pytestmark = pytest.mark.gpu

F32_ABS = 1e-5

CASES = {
    # name: (Hq, Hkv, D, rotary_dim, theta, dtype, gated, norm)
    "qwen3.5-gated-partial": (16, 2, 256, 64, 1e7, "bf16", True, True),
    "qwen7b-rope-only": (28, 4, 128, 128, 1e6, "bf16", False, False),
    "qwen7b-norm": (28, 4, 128, 128, 1e6, "bf16", True, True),
    "d64-half": (14, 2, 64, 32, 1e4, "bf16", True, True),
    "d32-mha": (4, 4, 32, 32, 1e4, "bf16", False, True),
    "f32-d128": (8, 2, 128, 64, 1e6, "f32", True, True),
    "f32-d256-no-rope": (8, 1, 256, 0, 1e6, "f32", True, True),
    "f32-d32": (4, 2, 32, 16, 1e4, "f32", False, False),
    # rotary halves that are not a multiple of the 16-byte vector take the
    # workgroup-per-token kernel; a partner distance of 6 lanes (not a power of 2)
    "d128-rd8-narrow": (28, 4, 128, 8, 1e6, "bf16", True, True),
    "f32-d64-rd4-narrow": (14, 2, 64, 4, 1e4, "f32", False, True),
    "d128-rd96": (28, 4, 128, 96, 1e6, "bf16", True, True),
    "d256-f32-full": (8, 1, 256, 256, 1e4, "f32", False, True),
}


def _i32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _f32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def _close(got, ref, dtype, what):
    """got, ref in the pool dtype's storage (last axis = one head row).
    bf16: |got - ref| <= one bf16 ulp of ref + 1e-5 * the row's max |ref|
    (the second term covers cancellation in x1*cos - x2*sin, where f32
    errors are relative to the operands, not to the difference)."""
    if dtype == "f32":
        err = float(np.max(np.abs(got.astype(np.float64) - ref), initial=0.0))
        assert err <= F32_ABS, f"{what}: max-abs error {err:.3e} > {F32_ABS}"
        return
    g, r = orc.bf16_to_f32(got).astype(np.float64), orc.bf16_to_f32(ref).astype(np.float64)
    tol = np.spacing(np.abs(r).astype(np.float32)).astype(np.float64) * 65536.0
    tol = tol + 1e-5 * np.max(np.abs(r), axis=-1, keepdims=True)
    bad = np.abs(g - r) > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements beyond tolerance, worst "
                           f"{float(np.max(np.abs(g - r) - tol)):.3e} past it")
    same = float(np.mean(got == ref)) if got.size else 1.0
    assert same >= 0.99, f"{what}: only {same:.4f} of elements bit-identical"


def _run_case(name, n, seed, slots=None, positions=None):
    Hq, Hkv, D, rd, theta, dtype, gated, norm = CASES[name]
    nb = max(8, (n + 15) // 16 * 2)
    desc = PoolDesc(2, Hkv, Hq, D, nb, dtype)
    rng = np.random.default_rng(seed)
    base = rng.standard_normal(desc.shape).astype(np.float32)
    host = base if dtype == "f32" else orc.f32_to_bf16(base)
    qshape = (n, Hq, 2, D) if gated else (n, Hq, D)
    q = (rng.standard_normal(qshape) * 2).astype(np.float32)
    k = (rng.standard_normal((n, Hkv, D)) * 2).astype(np.float32)
    v = rng.standard_normal((n, Hkv, D)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = (orc.f32_to_bf16(a) for a in (q, k, v))
    wq = rng.uniform(-0.5, 0.5, D).astype(np.float32) if norm else None
    wk = rng.uniform(-0.5, 0.5, D).astype(np.float32) if norm else None
    f = rope_inv_freq(rd, theta) if rd else None
    if slots is None:
        slots = rng.permutation(nb * 16)[:n].astype(np.int32)
    if positions is None:
        positions = rng.integers(0, 32768, n).astype(np.int32)
    layer = 1
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        qo = pool.qk_norm_rope_append(layer, to_device(q), to_device(k), to_device(v), _i32(positions),
                                      _i32(slots), None if wq is None else _f32(wq),
                                      None if wk is None else _f32(wk), None if f is None else _f32(f),
                                      eps=1e-6, gated=gated)
        pool.check()
        got_q, got_pool = to_host(qo), pool.read()
    ref_pool = host.copy()
    ref_q = orc.qk_norm_rope_append(odesc(desc), ref_pool, layer, widen(q), widen(k), widen(v), wq, wk, f,
                                    1e-6, positions, slots)
    return got_q, got_pool, ref_q, ref_pool, slots, dtype


@pytest.mark.parametrize("name", list(CASES))
def test_prep_matches_oracle(name):
    got_q, got_pool, ref_q, ref_pool, slots, dtype = _run_case(name, 37, 5)
    _close(got_q, ref_q, dtype, "q")
    blk, off = slots // 16, slots % 16
    # v rows bit-exact; every row the step does not write bit-exact
    assert np.array_equal(got_pool[1, 1, blk, off], ref_pool[1, 1, blk, off])
    _close(got_pool[1, 0, blk, off], ref_pool[1, 0, blk, off], dtype, "k rows")
    mask = np.ones(got_pool.shape[:4], bool)
    mask[1, 0, blk, off] = False
    assert np.array_equal(got_pool[mask], ref_pool[mask])


def test_prep_prefill_sized_batch():
    """A 2048-token prompt chunk at consecutive positions and slots."""
    n = 2048
    got_q, got_pool, ref_q, ref_pool, slots, dtype = _run_case(
        "qwen7b-norm", n, 6, slots=np.arange(16, 16 + n, dtype=np.int32),
        positions=np.arange(n, dtype=np.int32))
    _close(got_q, ref_q, dtype, "q")
    assert np.array_equal(got_pool[:, 1], ref_pool[:, 1])
    _close(got_pool[1, 0], ref_pool[1, 0], dtype, "k plane")


def test_prep_position_zero_is_norm_only():
    """At position 0 the rotation is the identity: the result equals the
    no-RoPE launch bit for bit."""
    import torch

    Hq, Hkv, D = 8, 2, 128
    desc = PoolDesc(1, Hkv, Hq, D, 4, "bf16")
    rng = np.random.default_rng(7)
    q = to_device(orc.f32_to_bf16(rng.standard_normal((5, Hq, 2, D)).astype(np.float32)))
    k = to_device(orc.f32_to_bf16(rng.standard_normal((5, Hkv, D)).astype(np.float32)))
    v = torch.zeros_like(k)
    w = _f32(rng.uniform(-0.5, 0.5, D))
    with DeviceKvPool(desc) as pool:
        pool.write(np.zeros(desc.shape, np.uint16))
        zeros = _i32(np.zeros(5))
        a = to_host(pool.qk_norm_rope_append(0, q, k, v, zeros, _i32(np.arange(5)), w, w,
                                             _f32(rope_inv_freq(D, 1e6))))
        b = to_host(pool.qk_norm_rope_append(0, q, k, v, zeros, _i32(np.arange(5) + 5), w, w, None))
        pool.check()
        p = pool.read()
    assert np.array_equal(a, b)
    assert np.array_equal(p[0, 0, 0, :5], p[0, 0, 0, 5:10])


def test_prep_unaligned_weights():
    """Norm weights at a 4-byte offset (not 16-byte aligned) take the
    workgroup-per-token kernel; both launches agree with the oracle."""
    import torch

    Hq, Hkv, D, n = 28, 4, 128, 9
    desc = PoolDesc(1, Hkv, Hq, D, 4, "bf16")
    rng = np.random.default_rng(9)
    q = orc.f32_to_bf16(rng.standard_normal((n, Hq, 2, D)).astype(np.float32))
    k = orc.f32_to_bf16(rng.standard_normal((n, Hkv, D)).astype(np.float32))
    v = orc.f32_to_bf16(rng.standard_normal((n, Hkv, D)).astype(np.float32))
    w = rng.uniform(-0.5, 0.5, D).astype(np.float32)
    f = rope_inv_freq(D, 1e6)
    pos, slots = rng.integers(0, 9000, n).astype(np.int32), np.arange(n, dtype=np.int32)
    buf = torch.zeros(D + 1, dtype=torch.float32, device="cuda")
    buf[1:] = torch.from_numpy(w).cuda()
    outs = []
    for wt in (_f32(w), buf[1:]):
        with DeviceKvPool(desc) as pool:
            pool.write(np.zeros(desc.shape, np.uint16))
            qo = pool.qk_norm_rope_append(0, to_device(q), to_device(k), to_device(v), _i32(pos), _i32(slots),
                                          wt, wt, _f32(f))
            pool.check()
            outs.append((to_host(qo), pool.read()))
    ref_pool = np.zeros(desc.shape, np.uint16)
    ref_q = orc.qk_norm_rope_append(odesc(desc), ref_pool, 0, widen(q), widen(k), widen(v), w, w, f, 1e-6,
                                    pos, slots)
    for got_q, got_pool in outs:
        _close(got_q, ref_q, "bf16", "q")
        _close(got_pool[0, 0], ref_pool[0, 0], "bf16", "k plane")
        assert np.array_equal(got_pool[0, 1], ref_pool[0, 1])


def test_prep_bad_slot_is_reported_and_skipped():
    Hq, Hkv, D = 8, 2, 64
    desc = PoolDesc(1, Hkv, Hq, D, 2, "bf16")
    rng = np.random.default_rng(8)
    host = orc.f32_to_bf16(rng.standard_normal(desc.shape).astype(np.float32))
    q = orc.f32_to_bf16(rng.standard_normal((3, Hq, 2, D)).astype(np.float32))
    k = orc.f32_to_bf16(rng.standard_normal((3, Hkv, D)).astype(np.float32))
    v = orc.f32_to_bf16(rng.standard_normal((3, Hkv, D)).astype(np.float32))
    slots = np.array([3, 32, 7], np.int32)  # 32 is past the 2-block pool
    pos = np.array([1, 2, 3], np.int32)
    w = rng.uniform(-0.5, 0.5, D).astype(np.float32)
    f = rope_inv_freq(D, 1e4)
    with DeviceKvPool(desc) as pool:
        pool.write(host)
        qo = pool.qk_norm_rope_append(0, to_device(q), to_device(k), to_device(v), _i32(pos), _i32(slots),
                                      _f32(w), _f32(w), _f32(f))
        with pytest.raises(DeviceIndexError) as ei:
            pool.check()
        assert ei.value.bits & dp.DEVERR_SLOT
        got_q, got_pool = to_host(qo), pool.read()
    ref_pool = host.copy()
    keep = [0, 2]
    ref_q = orc.qk_norm_rope_append(odesc(desc), ref_pool, 0, widen(q)[keep], widen(k)[keep], widen(v)[keep],
                                    w, w, f, 1e-6, pos[keep], slots[keep])
    _close(got_q[keep], ref_q, "bf16", "q")  # q rows do not depend on the slot
    assert np.array_equal(got_pool[0, 1], ref_pool[0, 1])
    _close(got_pool[0, 0], ref_pool[0, 0], "bf16", "k plane")


def test_prep_argument_errors():
    import torch

    desc = PoolDesc(1, 2, 8, 128, 4, "bf16")
    with DeviceKvPool(desc) as pool:
        q = torch.zeros((2, 8, 2, 128), dtype=torch.bfloat16, device="cuda")
        k = torch.zeros((2, 2, 128), dtype=torch.bfloat16, device="cuda")
        w = _f32(np.zeros(128))
        pos, sl = _i32([0, 1]), _i32([0, 1])
        with pytest.raises(BackendError):  # rotary_dim 6 is not a multiple of 2 * 128/64
            pool.qk_norm_rope_append(0, q, k, k, pos, sl, w, w, _f32(np.ones(3)))
        with pytest.raises(BackendError):  # rotary_dim past head_dim
            pool.qk_norm_rope_append(0, q, k, k, pos, sl, w, w, _f32(np.ones(66)))
        with pytest.raises(BackendError):  # layer out of range
            pool.qk_norm_rope_append(1, q, k, k, pos, sl, w, w, None)
        with pytest.raises(BackendError):  # one weight only
            pool.qk_norm_rope_append(0, q, k, k, pos, sl, w, None, None)
        with pytest.raises(BackendError):  # ungated q shape given as gated
            pool.qk_norm_rope_append(0, q[:, :, 0].contiguous(), k, k, pos, sl, w, w, None)
        pool.qk_norm_rope_append(0, q[:0], k[:0], k[:0], pos[:0], sl[:0], w, w, None)  # no tokens: no-op
        pool.check()
