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
