"""Shared test helpers: seeded pools, uploads, tolerance checks."""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc

F32_MAX_ABS = 1e-5   # f32 attention: max-abs error against the f32 oracle
BF16_REL = 2e-2      # bf16 attention: per-row max error / per-row max |ref|


def odesc(desc):
    """oracle descriptor of a mitten_amd.PoolDesc."""
    return orc.desc(desc.num_layers, desc.num_kv_heads, desc.head_dim, desc.num_blocks,
                    desc.elem_bytes, desc.page_size)


def normal(seed: int, shape, dtype: str) -> np.ndarray:
    """N(0,1) values as the pool dtype's host representation (f32 or bf16 bits)."""
    x = np.random.default_rng(seed).standard_normal(int(np.prod(shape)), dtype=np.float32)
    x = x.reshape(shape)
    return x if dtype == "f32" else orc.f32_to_bf16(x)


def widen(x: np.ndarray) -> np.ndarray:
    return x if x.dtype == np.float32 else orc.bf16_to_f32(x)


def to_device(x: np.ndarray, dtype: str | None = None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x))
    if x.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.cuda()


def to_host(t) -> np.ndarray:
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bits(x: np.ndarray) -> np.ndarray:
    """Raw bit view for bit-exact comparison (NaN-safe)."""
    return x.view(np.uint32) if x.dtype == np.float32 else x.view(np.uint16)


def assert_attention_close(got: np.ndarray, ref: np.ndarray, dtype: str) -> float:
    """got: device output on host (f32 or bf16 bits); ref: f32 oracle output.
    f32: max |got - ref| <= 1e-5.  bf16: for every (sequence, head) row,
    max |got - ref| <= 2e-2 * max |ref|. Returns the observed metric."""
    g = widen(got).astype(np.float64)
    r = ref.astype(np.float64)
    assert np.all(np.isfinite(g)), "non-finite attention output"
    if dtype == "f32":
        err = float(np.max(np.abs(g - r)))
        assert err <= F32_MAX_ABS, f"max-abs error {err:.3e} > {F32_MAX_ABS}"
        return err
    rowerr = np.max(np.abs(g - r), axis=-1) / np.maximum(np.max(np.abs(r), axis=-1), 1e-30)
    worst = float(rowerr.max())
    assert worst <= BF16_REL, f"row-relative error {worst:.3e} > {BF16_REL}"
    return worst
