"""Pins of the oracle's fused pre-attention step (q/k RMSNorm with weight
1 + w, partial NeoX RoPE, append; inference-model-qwen/src/model.rs:104-108,
371-392, 508-540) and of the host-side RoPE frequency table.

What pins it: hand-computed known answers; a float64 restatement in another
form (the half-rotation as multiplication by a unit complex number, the norm
through numpy's library mean); closed forms (position 0 is the identity,
dims past rotary_dim pass through, a rotation keeps each pair's norm, scores
depend on positions only through their difference); and mistakes planted in
a copy of the float64 restatement (GPT-J interleaved pairs, a flipped sign,
w instead of 1 + w, eps dropped, a sum instead of the mean, rotation over the
whole head) that each move the result far outside the tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from mitten_amd.device_pool import rope_inv_freq
from oracle import oracle as orc

TOL = 2e-5  # f32 oracle against the float64 restatement, values of order 1


def _np_norm_rope(x, w, eps, inv_freq, pos, *, pairs="neox", sign=1.0, one_plus_w=True, use_eps=True,
                  mean=True, rotate_all=False):
    """float64 restatement: RMSNorm(1 + w), then rotation of the pairs by
    e^{i a}, a = (f32) pos * inv_freq (the reference forms the angle in f32,
    model.rs:517-520). Keyword arguments plant mistakes."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    if w is not None:
        ms = np.mean(x * x, axis=-1, keepdims=True) if mean else np.sum(x * x, axis=-1, keepdims=True)
        y = x / np.sqrt(ms + (np.float64(np.float32(eps)) if use_eps else 0.0))
        y = y * ((np.asarray(w, np.float64) + 1.0) if one_plus_w else np.asarray(w, np.float64))
    else:
        y = x.copy()
    if inv_freq is None or len(inv_freq) == 0:
        return y
    f = np.asarray(inv_freq, np.float32)
    half = f.size
    rd = D if rotate_all else 2 * half
    if rotate_all:  # the same frequencies spread over the whole head
        f = np.resize(f, D // 2)
        half = D // 2
    ang = (np.asarray(pos, np.float32)[..., None] * f).astype(np.float64)
    rot = np.exp(1j * sign * ang)
    out = y.copy()
    if pairs == "neox":
        z = (y[..., :half] + 1j * y[..., half:rd]) * rot
        out[..., :half], out[..., half:rd] = z.real, z.imag
    else:  # GPT-J: pairs (2i, 2i + 1)
        z = (y[..., 0:rd:2] + 1j * y[..., 1:rd:2]) * rot
        out[..., 0:rd:2], out[..., 1:rd:2] = z.real, z.imag
    return out


def _rows(seed, n, D, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((n, D)) * scale).astype(np.float32)


def test_known_answers():
    # D=4, w=0, eps=0: x / rms(x) = [2,0,0,0]; rotate pair (0,2) by pos*inv_freq[0] = 1 rad
    got = orc.norm_rope_rows(np.array([[1, 0, 0, 0]], np.float32), np.zeros(4, np.float32), 0.0,
                             np.array([1.0, 1e-3], np.float32), [1])
    assert np.allclose(got[0], [2 * np.cos(1.0), 0, 2 * np.sin(1.0), 0], rtol=0, atol=3e-7)
    # D=2, norm only: mean(9, 16) = 12.5; weights 0.5 / -0.5 scale by 1.5 / 0.5
    got = orc.norm_rope_rows(np.array([[3, 4]], np.float32), np.array([0.5, -0.5], np.float32), 0.0, None, [7])
    assert np.allclose(got[0], [3 / np.sqrt(12.5) * 1.5, 4 / np.sqrt(12.5) * 0.5], rtol=2e-7, atol=0)
    # rotary_dim 2 of 4, by pi/2: pair (0, 1) -> (-x1, x0), dims 2, 3 pass through
    got = orc.norm_rope_rows(np.array([[1.0, 2.0, 3.0, 4.0]], np.float32), None, 0.0,
                             np.array([np.pi / 2], np.float32), [1])
    assert np.allclose(got[0], [-2.0, 1.0, 3.0, 4.0], atol=3e-7)


@pytest.mark.parametrize("D,rd,theta,eps", [(128, 128, 1e6, 1e-6), (256, 64, 1e7, 1e-6), (64, 32, 1e4, 1e-5),
                                             (32, 32, 1e4, 0.5)])
def test_against_float64_complex_restatement(D, rd, theta, eps):
    n = 300
    x = _rows(1, n, D, 3.0)
    w = np.random.default_rng(2).uniform(-0.5, 0.5, D).astype(np.float32)
    f = rope_inv_freq(rd, theta)
    pos = np.random.default_rng(3).integers(0, 40000, n).astype(np.int32)
    got = orc.norm_rope_rows(x, w, eps, f, pos)
    ref = _np_norm_rope(x, w, eps, f, pos)
    assert np.max(np.abs(got - ref)) < TOL


def test_closed_forms():
    D, rd = 128, 64
    x = _rows(4, 50, D)
    w = np.random.default_rng(5).uniform(-0.5, 0.5, D).astype(np.float32)
    f = rope_inv_freq(rd, 1e6)
    normed = orc.norm_rope_rows(x, w, 1e-6, None, np.zeros(50, np.int32))
    # position 0 rotates by cos 0 = 1, sin 0 = 0: bit-identical to the norm alone
    at0 = orc.norm_rope_rows(x, w, 1e-6, f, np.zeros(50, np.int32))
    assert np.array_equal(at0.view(np.uint32), normed.view(np.uint32))
    pos = np.arange(50, dtype=np.int32) * 997
    y = orc.norm_rope_rows(x, w, 1e-6, f, pos)
    # dims past rotary_dim pass through unchanged
    assert np.array_equal(y[:, rd:].view(np.uint32), normed[:, rd:].view(np.uint32))
    # each rotated pair keeps its norm
    h = rd // 2
    n_in = np.hypot(normed[:, :h].astype(np.float64), normed[:, h:rd])
    n_out = np.hypot(y[:, :h].astype(np.float64), y[:, h:rd])
    assert np.max(np.abs(n_in - n_out)) < 1e-5
    # w = 0, eps = 0: unit mean square
    unit = orc.norm_rope_rows(x, np.zeros(D, np.float32), 0.0, f, pos)
    assert np.allclose(np.mean(unit.astype(np.float64) ** 2, axis=-1), 1.0, atol=1e-5)
    # eps counts: tiny rows come out with mean square var / (var + eps)
    tiny = x * np.float32(1e-3)
    t = orc.norm_rope_rows(tiny, np.zeros(D, np.float32), 1e-6, None, np.zeros(50, np.int32))
    var = np.mean(tiny.astype(np.float64) ** 2, axis=-1)
    assert np.allclose(np.mean(t.astype(np.float64) ** 2, axis=-1), var / (var + np.float32(1e-6)), rtol=1e-5)


def test_scores_depend_only_on_relative_position():
    """RoPE's defining property: <R(q, m), R(k, n)> = <R(q, m + s), R(k, n + s)>."""
    D = 64
    f = rope_inv_freq(D, 1e4)
    q, k = _rows(6, 1, D), _rows(7, 1, D)
    dots = []
    for s in (0, 5, 40, 300):
        rq = orc.norm_rope_rows(q, None, 0.0, f, [10 + s]).astype(np.float64)
        rk = orc.norm_rope_rows(k, None, 0.0, f, [3 + s]).astype(np.float64)
        dots.append(float((rq @ rk.T)[0, 0]))
    assert np.allclose(dots, dots[0], rtol=1e-4, atol=1e-4)
    far = orc.norm_rope_rows(k, None, 0.0, f, [4]).astype(np.float64)
    rq = orc.norm_rope_rows(q, None, 0.0, f, [10]).astype(np.float64)
    assert abs(float((rq @ far.T)[0, 0]) - dots[0]) > 1e-3  # and they do depend on it


def test_inv_freq_table():
    for rd, theta in ((128, 1e6), (64, 1e7), (32, 1e4)):
        f = rope_inv_freq(rd, theta)
        assert f.dtype == np.float32 and f.size == rd // 2 and f[0] == 1.0
        exact = theta ** (-2.0 * np.arange(rd // 2) / rd)
        assert np.max(np.abs(f / exact - 1.0)) < 1e-5
        assert np.all(np.diff(f) < 0)


def test_checks_detect_planted_mistakes():
    D, rd = 128, 64
    x = _rows(8, 64, D, 0.05)
    w = np.random.default_rng(9).uniform(-0.5, 0.5, D).astype(np.float32)
    f = rope_inv_freq(rd, 1e4)
    pos = np.random.default_rng(10).integers(1, 4000, 64).astype(np.int32)
    eps = 1e-3
    good = orc.norm_rope_rows(x, w, eps, f, pos)
    assert np.max(np.abs(good - _np_norm_rope(x, w, eps, f, pos))) < TOL
    wrong = {
        "GPT-J interleaved pairs": dict(pairs="gptj"),
        "rotation sign flipped": dict(sign=-1.0),
        "w instead of 1 + w": dict(one_plus_w=False),
        "eps dropped": dict(use_eps=False),
        "sum of squares, not mean": dict(mean=False),
        "whole head rotated": dict(rotate_all=True),
    }
    for name, kw in wrong.items():
        assert np.max(np.abs(good - _np_norm_rope(x, w, eps, f, pos, **kw))) > 1e-3, name


@pytest.mark.parametrize("es", [4, 2])
def test_fused_step_appends_prepared_k_and_raw_v(es):
    """The fused step's pool effect equals append of (normed, rotated k, v) and
    its q output is the normed, rotated q half of the gated projection."""
    Hq, Hkv, D, nb = 4, 2, 64, 6
    d = orc.desc(2, Hkv, D, nb, es)
    shape = orc.pool_shape(d)
    base = np.random.default_rng(11).standard_normal(int(np.prod(shape))).astype(np.float32).reshape(shape)
    pool = base if es == 4 else orc.f32_to_bf16(base)
    n = 5
    rng = np.random.default_rng(12)
    qg = rng.standard_normal((n, Hq, 2, D)).astype(np.float32)
    k = rng.standard_normal((n, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((n, Hkv, D)).astype(np.float32)
    if es == 2:
        qg, k, v = (orc.bf16_to_f32(orc.f32_to_bf16(a)) for a in (qg, k, v))
    wq = rng.uniform(-0.3, 0.3, D).astype(np.float32)
    wk = rng.uniform(-0.3, 0.3, D).astype(np.float32)
    f = rope_inv_freq(32, 1e6)
    pos = np.array([0, 1, 17, 300, 5000], np.int32)
    slots = np.array([3, 40, 17, 95, 64], np.int32)
    after = pool.copy()
    qo = orc.qk_norm_rope_append(d, after, 1, qg, k, v, wq, wk, f, 1e-6, pos, slots)
    exp_q = orc.norm_rope_rows(qg[:, :, 0], wq, 1e-6, f, np.repeat(pos, Hq))
    exp_k = orc.norm_rope_rows(k, wk, 1e-6, f, np.repeat(pos, Hkv))
    expect = pool.copy()
    cast = (lambda a: a) if es == 4 else orc.f32_to_bf16
    for t, s in enumerate(slots):
        expect[1, 0, s // 16, s % 16] = cast(exp_k[t])
        expect[1, 1, s // 16, s % 16] = cast(v[t])
    assert np.array_equal(after, expect)
    assert np.array_equal(qo, cast(exp_q))
    with pytest.raises(ValueError):
        orc.qk_norm_rope_append(d, after, 1, qg, k, v, wq, wk, f, 1e-6, pos, np.array([0, 1, 2, 3, 96], np.int32))
