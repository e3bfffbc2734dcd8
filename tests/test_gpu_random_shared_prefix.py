"""Seeded random decode steps over a shared prefix: random head shapes,
sequence counts, prefix lengths (whole blocks plus a partial one), suffix
ranges, piece counts and the zero sink, each against the oracle's decode
attention over the whole tables with the fused append bit-exact (the checks
of tests/test_gpu_shared_prefix.py's cases, on random sizes)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import assert_attention_close
from tests.test_gpu_shared_prefix import SHAPES, _case

pytestmark = pytest.mark.gpu

N_CASES = 16


def _params(i: int):
    rng = np.random.default_rng(5000 + i)
    shape = list(SHAPES)[int(rng.integers(len(SHAPES)))]
    seqs = int(rng.integers(1, 161))
    prefix = int(rng.integers(16, 1501))
    lo = int(rng.integers(1, 150))
    hi = lo + int(rng.integers(0, 300))
    pieces = [0, 0, int(rng.integers(1, 600))][int(rng.integers(3))]
    return shape, seqs, prefix, lo, hi, pieces, bool(rng.integers(2)), 5100 + 10 * i


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shared_prefix_step_matches_the_oracle(i):
    shape, seqs, prefix, lo, hi, pieces, zero_sink, seed = _params(i)
    print(f"case {i}: {shape} seqs {seqs} prefix {prefix} suffixes {lo}..{hi} pieces {pieces} "
          f"zero_sink {zero_sink}", flush=True)
    outs, ref = _case(shape, seqs, prefix, lo, hi, seed, zero_sink=zero_sink, pieces=pieces)
    assert_attention_close(outs[0], ref, "bf16")
