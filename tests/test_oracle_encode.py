"""Pins of oracle/encode.py (the exhaustive nearest-codeword scan)."""

import numpy as np
import pytest

from oracle import e8p
from oracle import encode as oenc


@pytest.mark.parametrize("code_bits", [8, 16])
def test_every_codeword_encodes_to_itself(code_bits):
    g = oenc.grid(code_bits)
    assert len(np.unique(g, axis=0)) == len(g)
    np.testing.assert_array_equal(oenc.nearest(g, code_bits), np.arange(len(g)))
    w = np.abs(np.random.default_rng(code_bits).standard_normal(8)).astype(np.float32) + 0.05
    np.testing.assert_array_equal(oenc.nearest(g, code_bits, w), np.arange(len(g)))


def _exact_argmin(v8, g8, wi):
    """Argmin of exact integer distances (inputs scaled by 8 to integers), ties to the lowest index."""
    d = (((v8[:, None, :] - g8[None, :, :]) ** 2) * wi).sum(-1)
    return d.argmin(axis=1)  # first occurrence: the lowest index


@pytest.mark.parametrize("code_bits", [8, 16])
def test_dyadic_inputs_match_exact_integer_argmin(code_bits):
    g = oenc.grid(code_bits)
    rng = np.random.default_rng(5)
    lo = g[rng.integers(0, len(g) - 1, 120)]
    mid = ((lo + g[np.minimum(rng.integers(0, len(g), 120), len(g) - 1)]) / 2).astype(np.float32)
    m = min(120, len(g) - 1)
    adj = ((g[:m] + g[1:m + 1]) / 2).astype(np.float32)  # adjacent rows: exact ties
    v = np.concatenate([mid, adj, np.full((4, 8), 0.25, np.float32), np.zeros((4, 8), np.float32)])
    g8 = np.rint(g.astype(np.float64) * 8).astype(np.int64)
    v8 = np.rint(v.astype(np.float64) * 8).astype(np.int64)
    assert (v8 == v * 8).all() and (g8 == g * 8).all()
    for wi in (np.ones(8, np.int64), np.array([1, 2, 3, 1, 2, 3, 1, 0], np.int64)):
        want = np.concatenate([_exact_argmin(v8[i:i + 64], g8, wi) for i in range(0, len(v8), 64)])
        np.testing.assert_array_equal(oenc.nearest(v, code_bits, wi.astype(np.float32)), want)


def test_random_inputs_match_a_float64_argmin_and_per_row_weights():
    g = oenc.grid(16).astype(np.float64)
    rng = np.random.default_rng(9)
    v = (rng.standard_normal((200, 8)) * 0.6).astype(np.float32)
    w = (np.abs(rng.standard_normal((200, 8))) + 0.05).astype(np.float32)
    d = ((v[:, None, :].astype(np.float64) - g[None]) ** 2 * w[:, None, :].astype(np.float64)).sum(-1)
    np.testing.assert_array_equal(oenc.nearest(v, 16, w), d.argmin(1))
    shared = oenc.nearest(v, 16, w[0])
    np.testing.assert_array_equal(shared, oenc.nearest(v, 16, np.broadcast_to(w[0], v.shape)))


def test_quantize_scale_divisor_is_the_grids_largest_magnitude():
    assert np.abs(oenc.grid(16)).max() == np.float32(np.abs(e8p.e8p_abs_grid()).max() + 0.25) == 2.75
    assert np.abs(oenc.grid(8)).max() == np.abs(e8p.decode_e8_1bit(np.arange(256, dtype=np.uint8))).max()
    w = np.zeros((2, 16), np.float32)
    w[1, 3] = 2.75
    codes, scales = oenc.quantize_weight_rtn(w, group_size=16, code_bits=16)
    assert scales.tolist() == [[0.0], [1.0]]  # a zero group keeps scale 0 (it divided by 1)
    np.testing.assert_array_equal(codes, oenc.nearest(w.reshape(-1, 8), 16).reshape(2, 2))


def _rtn_vectors(n, code_bits, seed, group=512):
    """Vectors as the RTN feeds them to the search: Gaussian rows divided by max |w| / the grid's largest value."""
    w = np.random.default_rng(seed).standard_normal((n * 8 // group, group)).astype(np.float32)
    div = np.float32(np.abs(oenc.grid(code_bits)).max())
    s = (np.abs(w).max(axis=1) / div).astype(np.float32)
    return (w / s[:, None]).astype(np.float32).reshape(-1, 8)


@pytest.mark.parametrize("code_bits", [8, 16])
def test_float32_search_restatement_pins(code_bits):
    """The float32 restatement of the reference's searches returns every
    codeword's own code, and on dyadic inputs (exact in float32) without a tie
    the exact scan's code."""
    g = oenc.grid(code_bits)
    np.testing.assert_array_equal(oenc.nearest_f32(g, code_bits), np.arange(len(g)))
    rng = np.random.default_rng(3)
    v = (rng.integers(-24, 25, (4000 if code_bits == 8 else 800, 8)) / 8.0).astype(np.float32)
    v64, g64 = v.astype(np.float64), g.astype(np.float64)
    # exact in float64: every term is a multiple of 1/32 below 2^10
    d = (v64 * v64).sum(1)[:, None] + (g64 * g64).sum(1)[None, :] - 2 * v64 @ g64.T
    part = np.partition(d, 1, axis=1)
    clear = part[:, 1] > part[:, 0]
    assert clear.sum() > len(v) // 4
    np.testing.assert_array_equal(oenc.nearest_f32(v[clear], code_bits), d[clear].argmin(1))


@pytest.mark.parametrize("code_bits,n", [(8, 1_000_000), (16, 65536)])
def test_float32_search_agrees_with_the_exact_scan(code_bits, n):
    """Agreement of the reference's float32 search with the exact scan on RTN
    inputs: 8-bit, 0 of 1e6 differ; E8P, 2 of 1e6 differ (measured once over
    1e6; this test takes 65,536). Every difference is a near-tie: the float32
    pick is farther by at most 1e-6 (|v|^2 + 1) in exact distance."""
    v = _rtn_vectors(n, code_bits, seed=11)
    ex, f = oenc.nearest(v, code_bits), oenc.nearest_f32(v, code_bits)
    dis = np.flatnonzero(ex != f)
    assert dis.size <= max(2, n // 10000)
    g = oenc.grid(code_bits).astype(np.float64)
    vv = v[dis].astype(np.float64)
    gap = ((vv - g[f[dis]]) ** 2).sum(1) - ((vv - g[ex[dis]]) ** 2).sum(1)
    assert ((gap >= 0) & (gap <= 1e-6 * ((vv ** 2).sum(1) + 1))).all()
