"""Pins of the oracle's bfloat16 rounding (oracle/ops.py ``round_bf16``), the
rounding of h the decode kernels store: against torch's own float32 ->
bfloat16 conversion on every bf16 pattern with each low half that decides a
rounding (exact, ties, one ulp either side of a tie, the largest), and on
random float32 bit patterns; float64 inputs rounded once, checked against an
exact rational rounding, and on values a float32 detour would round twice the
wrong way."""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ops


def _same(a, b):
    return np.all((a == b) | (np.isnan(a) & np.isnan(b)))


@pytest.mark.parametrize("low", [0x0000, 0x8000, 0x7FFF, 0x8001, 0x0001, 0xFFFF])
def test_float32_patterns_match_torch(low):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    f = (hi | low).view(np.float32)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).double().numpy()
    assert _same(ops.round_bf16(f), want)


def test_random_float32_patterns_match_torch():
    f = np.random.default_rng(7).integers(0, 1 << 32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).double().numpy()
    assert _same(ops.round_bf16(f), want)


def _nearest_bf16_exact(x: float) -> float:
    """Nearest bfloat16 by exact rationals, ties to the even significand (finite, normal range)."""
    q = Fraction(x)
    e = abs(q).numerator.bit_length() - abs(q).denominator.bit_length()
    if Fraction(2) ** e > abs(q):
        e -= 1
    step = Fraction(2) ** (max(e, -126) - 7)
    n, rem = divmod(q, step)
    if rem * 2 > step or (rem * 2 == step and n % 2 == 1):
        n += 1
    return float(n * step)


def test_float64_rounds_once_like_exact_rationals():
    rng = np.random.default_rng(8)
    x = rng.standard_normal(4000) * np.exp2(rng.integers(-60, 60, 4000))
    got = ops.round_bf16(x)
    want = np.array([_nearest_bf16_exact(float(v)) for v in x])
    np.testing.assert_array_equal(got, want)


def test_float64_just_past_a_tie_is_not_rounded_twice():
    # v = an even bf16 value + half its step + a sliver: the nearest bf16 is the next one up. Through
    # float32 first, the sliver is lost, the tie goes to even, and the result is one step low.
    rng = np.random.default_rng(9)
    with np.errstate(invalid="ignore"):
        base = (rng.integers(0, 1 << 15, 1000, dtype=np.uint32) << 17).view(np.float32).astype(np.float64)  # even
    base = base[np.isfinite(base) & (np.abs(base) > 2.0 ** -120) & (np.abs(base) < 2.0 ** 120)]
    _, ex = np.frexp(base)
    step = np.ldexp(1.0, ex - 8)
    v = base + np.sign(base) * (step / 2 + step * 2.0 ** -30)
    assert (v.astype(np.float32).astype(np.float64) == base + np.sign(base) * step / 2).all()  # f32 sees a tie
    np.testing.assert_array_equal(ops.round_bf16(v), base + np.sign(base) * step)
    np.testing.assert_array_equal(ops.round_bf16(v.astype(np.float32)), base)  # the double rounding


def test_specials():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, ops.BF16_MAX, -ops.BF16_MAX, 3.4e38, 2.0 ** -133,
                  2.0 ** -134, 3 * 2.0 ** -135, 1e-300])
    got = ops.round_bf16(x)
    want = [0.0, -0.0, np.inf, -np.inf, np.nan, ops.BF16_MAX, -ops.BF16_MAX, np.inf, 2.0 ** -133, 0.0,
            2.0 ** -133, 0.0]
    assert _same(got, np.array(want))
    assert np.signbit(got[1])
