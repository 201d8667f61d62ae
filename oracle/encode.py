"""Nearest-codeword encoding and the data-free RTN quantiser -- CPU oracle
(test infrastructure only; see ``oracle/__init__.py``).

``nearest`` is the exhaustive weighted scan of ``cpu_ref.c`` (double
precision, the tree order stated there, ties to the lowest index): the
definition of the encoders' answer (``src/keep/quant/rtn.py:92-135``, the
exhaustive reference of ``tests/test_e8p_diagonal_hessian.py:14-19``).
``quantize_weight_rtn`` follows ``src/keep/quant/rtn.py:253-318``: per (row,
group) max |w| over the codebook's largest magnitude (fp32), a zero scale
divides by 1, each vector divided by its scale in fp32 and encoded.

Pins (``tests/test_oracle_encode.py``): every codeword of the E8P and 8-bit
grids encodes to itself; on dyadic inputs (grid midpoints, exact ties) with
integer weights the scan equals the argmin of exact integer distances, ties to
the lowest index; on random inputs it equals a float64 argmin computed another
way; the scale divisors equal the full grids' largest magnitudes.

``nearest_f32`` restates the reference's own float32 searches (the expanded
distance argmin of ``src/keep/vq/e8.py:255-280`` for the 8-bit table, the
factored E8P search of ``e8.py:290-366``). It is not an answer the encoders
must reproduce: the tests use it to count where float32 rounding makes the
reference pick another codeword than the exact scan, and to check that every
such case is a near-tie. Its pins: on exactly representable inputs far from
ties it returns the exact scan's codes (``tests/test_oracle_encode.py``).
"""

from __future__ import annotations

import numpy as np

from oracle import cpu, e8p


def grid(code_bits: int) -> np.ndarray:
    return e8p.e8p_full_grid() if code_bits == 16 else e8p.decode_e8_1bit(np.arange(256, dtype=np.uint8))


def nearest(vectors, code_bits: int, w=None) -> np.ndarray:
    return cpu.nearest(vectors, grid(code_bits), w)


def quantize_weight_rtn(weight, *, group_size: int, code_bits: int) -> tuple[np.ndarray, np.ndarray]:
    """``(codes [out, in/8], scales fp16 [out, groups])`` of the max_abs RTN."""

    w = np.asarray(weight, dtype=np.float32)
    out_dim, in_dim = w.shape
    groups = in_dim // group_size
    gv = w.reshape(out_dim, groups, group_size)
    divisor = np.float32(np.abs(grid(code_bits)).max())
    scales = (np.abs(gv).max(axis=2) / divisor).astype(np.float32)
    safe = np.where(scales > 0, scales, np.float32(1.0)).astype(np.float32)
    vec = gv.reshape(out_dim, groups, group_size // 8, 8) / safe[:, :, None, None]
    codes = nearest(vec.astype(np.float32), code_bits).reshape(out_dim, in_dim // 8)
    return codes.astype(np.uint16 if code_bits == 16 else np.uint8), scales.astype(np.float16)


def _popcount8(a: np.ndarray) -> np.ndarray:
    a = a.astype(np.uint32)
    n = np.zeros_like(a)
    for b in range(8):
        n += (a >> b) & 1
    return n


def _nearest_1bit_f32(v: np.ndarray) -> np.ndarray:
    """``|v|^2 + |c|^2 - 2 v.c`` in float32 over the 256-entry table, first minimum (``e8.py:267-278``)."""
    table = grid(8).astype(np.float32)
    vn = np.sum(v * v, axis=1)
    cn = np.sum(table * table, axis=1)
    d = (vn[:, None] + cn[None, :]) - (np.float32(2) * v) @ table.T
    return np.argmin(d, axis=1)


def _nearest_e8p_f32(v: np.ndarray) -> np.ndarray:
    """The factored E8P search in float32 (``e8.py:304-364``): per shift, the
    expanded distance to each of the 256 absolute rows, the signs that follow
    the target, and for an odd sign count the cheapest single flip
    (``4 |t_d| |r_d|``, first minimum) added to that row's distance; the first
    minimum over rows, the second shift taken only when strictly closer."""
    rows = e8p.e8p_abs_grid()
    absr = np.abs(rows)
    absn = np.sum(absr * absr, axis=1)
    bit = np.asarray([1 << s for s in e8p.E8P_SHUFFLE], dtype=np.uint32)  # output dim -> packed sign bit
    base = ((rows < 0).astype(np.uint32) * bit).sum(axis=1).astype(np.uint32)
    n = v.shape[0]
    at_n = np.arange(n)
    best = np.full(n, np.inf, dtype=np.float32)
    code = np.zeros(n, dtype=np.uint32)
    for parity, shift in ((0, np.float32(0.25)), (1, np.float32(-0.25))):
        t = v - shift
        at = np.abs(t)
        dist = (np.sum(at * at, axis=1)[:, None] + absn[None, :]) - (np.float32(2) * at) @ absr.T
        eff = ((t < 0).astype(np.uint32) * bit).sum(axis=1).astype(np.uint32)[:, None] ^ base[None, :]
        odd = (_popcount8(eff) & 1).astype(bool)
        pen = np.float32(4) * at[:, None, :] * absr[None, :, :]
        dist = np.where(odd, dist + pen.min(axis=2), dist)
        row = np.argmin(dist, axis=1)
        rd = dist[at_n, row]
        signs = eff[at_n, row]
        flip = bit[pen[at_n, row].argmin(axis=1)]
        signs = np.where(odd[at_n, row], signs ^ flip, signs) ^ parity
        take = rd < best
        best = np.where(take, rd, best)
        code = np.where(take, (row.astype(np.uint32) << 8) | signs, code)
    return code


def nearest_f32(vectors, code_bits: int, chunk: int = 8192) -> np.ndarray:
    """The reference's float32 nearest-codeword search (measurement only)."""
    v = np.asarray(vectors, dtype=np.float32).reshape(-1, 8)
    f = _nearest_1bit_f32 if code_bits == 8 else _nearest_e8p_f32
    return np.concatenate([f(v[i:i + chunk]) for i in range(0, v.shape[0], chunk)] or [np.zeros(0, np.int64)])
