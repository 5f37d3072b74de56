"""The oracle's model-dtype rounding against torch's casts, on the CPU.

oracle.model.bf16_round is the oracle's own round-to-nearest-even of fp32 to bfloat16 (integer arithmetic
on the bit pattern); every rounding point of the oracle goes through it, so it is pinned here against
torch's ``.to(torch.bfloat16)`` (what the reference's ``_silu_fp32`` / RMSNorm casts do) bit for bit: random
values over the whole exponent range, exact halfway cases with even and odd mantissas, the largest finite
values (which round to infinity), subnormals, signed zeros, infinities and NaN.  f16_round is numpy's cast,
checked the same way against torch's float16 cast."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.model import bf16_round, f16_round


def _cases(seed: int = 7) -> np.ndarray:
    rng = np.random.default_rng(seed)
    n = 1 << 20
    bits = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)  # every fp32 pattern, NaNs included
    mant = rng.standard_normal(n).astype(np.float32) * np.float32(10.0) ** rng.uniform(-40, 38, n).astype(np.float32)
    hi = rng.integers(0, 1 << 16, 4096, dtype=np.uint64).astype(np.uint32) << np.uint32(16)
    halfway = hi | np.uint32(0x8000)                  # exactly between two bf16 values, both parities of the mantissa
    near = np.concatenate([hi | np.uint32(0x7FFF), hi | np.uint32(0x8001)])
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, np.finfo(np.float32).max, -np.finfo(np.float32).max,
                        np.finfo(np.float32).tiny, 1e-45, -1e-45, 3.3895314e38, 1.0, -1.0], np.float32)
    return np.concatenate([bits.view(np.float32), mant, halfway.view(np.float32), near.view(np.float32), special])


def _same_bits(got: np.ndarray, want: np.ndarray) -> None:
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_round_matches_torch_cast():
    x = _cases()
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).to(torch.float32).numpy()
    _same_bits(bf16_round(x), want)


@pytest.mark.filterwarnings("ignore:overflow encountered in cast:RuntimeWarning")
def test_f16_round_matches_torch_cast():
    x = _cases(8)
    want = torch.from_numpy(x.copy()).to(torch.float16).to(torch.float32).numpy()
    _same_bits(f16_round(x), want)
