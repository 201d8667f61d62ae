"""Pins of oracle/block.py (the steps either side of the routed experts)."""

import math

import numpy as np
import pytest
import torch

from oracle import block


def _e4m3_grid() -> np.ndarray:
    """Every finite non-negative e4m3fn value (exponent bias 7, max 448), from the format's fields."""
    vals = [m / 8 * 2.0 ** -6 for m in range(8)]  # subnormals
    for e in range(1, 16):
        for m in range(8):
            if e == 15 and m == 7:
                continue  # NaN
            vals.append((1 + m / 8) * 2.0 ** (e - 7))
    return np.array(sorted(vals), dtype=np.float64)


def test_e4m3_grid_matches_torch():
    g = _e4m3_grid()
    assert g[-1] == 448.0 and len(g) == 127
    t = torch.from_numpy(g.astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(t, g.astype(np.float32))


def test_e4m3_round_matches_torch_on_every_bf16_value_and_every_tie():
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 448.0)]
    g = _e4m3_grid()
    ties = ((g[:-1] + g[1:]) / 2).astype(np.float32)  # exact in fp32: the midpoints need 5 significant bits
    near = np.concatenate([ties, np.nextafter(ties, np.float32(0)), np.nextafter(ties, np.float32(1e9))])
    rng = np.random.default_rng(0)
    rnd = (rng.standard_normal(200000) * np.exp(rng.uniform(-12, 6, 200000))).astype(np.float32)
    rnd = np.clip(rnd, -448, 448)
    for vals in (v, near, -near, rnd):
        want = torch.from_numpy(vals).to(torch.float8_e4m3fn).float().numpy()
        np.testing.assert_array_equal(block.e4m3_round(vals), want)


def test_pow2_ceil_closed_form():
    rng = np.random.default_rng(1)
    v = np.concatenate([np.exp(rng.uniform(-80, 80, 10000)), 2.0 ** np.arange(-100, 100)]).astype(np.float32)
    want = np.array([2.0 ** math.ceil(math.log2(float(a))) for a in v], dtype=np.float32)
    np.testing.assert_array_equal(block.pow2_ceil(v), want)


def test_rmsnorm_constant_rows_and_scale_invariance():
    n, eps = 256, 1e-6
    for c in (0.5, -3.0, 1e-3):
        g = np.linspace(-2, 2, n).astype(np.float32)
        y = block.rmsnorm(np.full((1, n), c, np.float32), g, eps)
        want = g * (c / math.sqrt(c * c + eps))
        np.testing.assert_allclose(y[0], want, rtol=2e-7, atol=0)
    x = np.random.default_rng(2).standard_normal((3, n)).astype(np.float32)
    base = block.rmsnorm(x, None, 0.0)
    for k in (-5, 3, 20):
        np.testing.assert_array_equal(block.rmsnorm(x * np.float32(2.0 ** k), None, 0.0), base)
    np.testing.assert_allclose((base.astype(np.float64) ** 2).mean(-1), 1.0, rtol=1e-6)


@pytest.mark.parametrize("pow2", [False, True])
@pytest.mark.parametrize("blk", [16, 128])
def test_act_quant_on_grid_within_half_step(pow2, blk):
    rng = np.random.default_rng(blk + pow2)
    y = (rng.standard_normal((4, 512)) * np.exp(rng.uniform(-6, 3, (4, 1)))).astype(np.float32)
    q = block.act_quant(y, blk, pow2)
    yb, qb = y.reshape(4, -1, blk), q.reshape(4, -1, blk)
    s = np.maximum(np.abs(yb).max(-1), 1e-4).astype(np.float32) * np.float32(1 / 448)
    if pow2:
        s = block.pow2_ceil(s)
        assert (block.act_quant(q, blk, pow2) == q).all(), "power-of-two scales: quantising twice changes nothing"
    grid = _e4m3_grid()
    # y / s (fp32) rounded to the nearest e4m3 value (brute force over the grid, ties to the even code),
    # times s in fp32, is q
    t = np.clip((yb / s[..., None]).astype(np.float32), -448, 448).astype(np.float64)
    dist = np.abs(np.abs(t)[..., None] - grid)
    best = dist.min(-1, keepdims=True)
    codes = np.arange(len(grid))
    pick = np.where(dist == best, codes % 2, 99).argmin(-1)  # ties sit between adjacent codes: take the even one
    e = np.copysign(grid[pick], t).astype(np.float32)
    np.testing.assert_array_equal(qb, (e * s[..., None]).astype(np.float32))


def test_shared_combine_order_and_rounding():
    r = np.array([1.0, 2.0 ** -10, 3.0, 2.0 ** 24], np.float32)
    s = np.array([2.0 ** 8, 1.0, -3.0, 1.0], np.float32)
    h = np.array([-2.0 ** 8, 1.0, 0.5, -2.0 ** 24], np.float32)
    out = block.shared_combine(r, s, h, "bfloat16")
    # 2 + 2^-10 rounds to 2 in bf16; routed + shared first: 2^24 + 1 is 2^24 in fp32, so the last sum is 0 (1 if
    # the residual were added to the routed sum first)
    np.testing.assert_array_equal(out, np.array([1.0, 2.0, 0.5, 0.0], np.float32))
    np.testing.assert_array_equal(block.shared_combine(r, None, None, "float32"), r)
