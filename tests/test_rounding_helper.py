"""CPU checks of tests.helpers.rounded, the oracle side of the GPU parity tests: FP64
values into float16 with one rounding, into bfloat16 through float32 (the kernels store
their FP64 results the same way)."""

from __future__ import annotations

import numpy as np
import torch

from tests.helpers import rounded


def test_float16_rounds_once_and_bfloat16_through_float32():
    one = 1.0
    past_f16 = one + 2.0**-11 + 2.0**-40  # float32 rounds it onto the float16 midpoint 1 + 2^-11
    assert float(rounded(np.array([past_f16]), torch.float16)[0]) == one + 2.0**-10
    assert float(rounded(np.array([one + 2.0**-11]), torch.float16)[0]) == one  # exact tie: even
    past_bf16 = one + 2.0**-8 + 2.0**-30
    assert float(rounded(np.array([past_bf16]), torch.bfloat16)[0]) == one  # through float32: the tie
    assert float(rounded(np.array([one + 2.0**-8 + 2.0**-20]), torch.bfloat16)[0]) == one + 2.0**-7
    assert float(rounded(np.array([-(one + 3 * 2.0**-8)]), torch.bfloat16)[0]) == -(one + 2 * 2.0**-7)


def test_float16_matches_brute_force_nearest():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(3000) * np.exp2(rng.integers(-12, 12, 3000))
    mids = (np.round(rng.standard_normal(1000) * 1024) + 0.5) / 1024 + rng.choice([-1, 1], 1000) * 2.0**-40
    x = np.concatenate([x, mids])
    got = rounded(x, torch.float16).double().numpy()
    grid = np.unique(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64))
    grid = grid[np.isfinite(grid)]
    hi = np.clip(np.searchsorted(grid, x), 1, grid.size - 1)
    lo_v, hi_v = grid[hi - 1], grid[hi]
    even_hi = (np.array(hi_v, dtype=np.float16).view(np.uint16) & 1) == 0
    pick_hi = (hi_v - x < x - lo_v) | ((hi_v - x == x - lo_v) & even_hi)
    np.testing.assert_array_equal(got, np.where(pick_hi, hi_v, lo_v))
