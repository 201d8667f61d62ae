"""Random-sign Walsh-Hadamard transform -- CPU oracle (test infrastructure).

Restated from the reference's ``src/keep/quant/rht.py:24-66``.

Pins: the FWHT is checked against ``scipy.linalg.hadamard`` (Sylvester order)
and by round-trip / norm preservation (``tests/test_glm45_air_rht.py:14-28``).
``deterministic_rht_signs`` is pinned by the FIPS 202 SHAKE256 known answer for
the empty message: the digest bytes, and the sign vector of ``seed=""`` derived
by hand from them (little-endian bit order, 0 -> -1), which a big-endian
unpack, a swapped sign map or another hash would each fail
(``tests/test_oracle_ops.py``).
"""

from __future__ import annotations

import hashlib
import math

import numpy as np


def _check_pow2(n: int) -> None:
    if n <= 0 or n & (n - 1):
        raise ValueError("RHT dimension must be a positive power of two")


def deterministic_rht_signs(dim: int, *, seed: int | str) -> np.ndarray:
    """+-1 int8 signs from ``shake_256(str(seed))`` (``rht.py:24-31``)."""

    _check_pow2(dim)
    raw = hashlib.shake_256(str(seed).encode("utf-8")).digest((dim + 7) // 8)
    bits = [(raw[i // 8] >> (i % 8)) & 1 for i in range(dim)]
    return np.array([1 if b else -1 for b in bits], dtype=np.int8)


def fwht(x: np.ndarray) -> np.ndarray:
    """Orthonormal fast Walsh-Hadamard transform over the last axis, float64
    (Sylvester order, ``rht.py:34-48``)."""

    v = np.array(x, dtype=np.float64, copy=True)
    n = v.shape[-1]
    _check_pow2(n)
    h = 1
    while h < n:
        v = v.reshape(v.shape[:-1] + (n // (2 * h), 2, h))
        a = v[..., 0, :].copy()
        b = v[..., 1, :].copy()
        v[..., 0, :] = a + b
        v[..., 1, :] = a - b
        v = v.reshape(v.shape[:-3] + (n,))
        h *= 2
    return v / math.sqrt(n)


def apply_rht(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``FWHT(x * signs)`` over the last axis (``rht.py:51-57``), float64."""

    s = np.asarray(signs, dtype=np.float64)
    return fwht(np.asarray(x, dtype=np.float64) * s)


def apply_inverse_rht(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``FWHT(x) * signs`` (``rht.py:60-66``), float64."""

    return fwht(x) * np.asarray(signs, dtype=np.float64)


def hadamard_f32(x: np.ndarray) -> np.ndarray:
    """The reference's float32 FWHT, ``_hadamard_np`` (``rht.py:34-48``): float32
    butterflies, width 1, 2, ..., n/2, then ``* float32(1 / sqrt(n))``. Every
    butterfly is one float32 add or subtract of the same two inputs in any
    schedule, so a GPU transform with this stage order matches it bit for bit.
    Pinned against the float64 ``fwht`` (Sylvester matrix) to float32 rounding."""

    v = np.array(x, dtype=np.float32, copy=True)
    n = v.shape[-1]
    _check_pow2(n)
    lead = v.shape[:-1]
    w = 1
    while w < n:
        v = v.reshape(lead + (n // (2 * w), 2, w))
        a = v[..., 0, :].copy()
        b = v[..., 1, :].copy()
        v[..., 0, :] = a + b
        v[..., 1, :] = a - b
        v = v.reshape(lead + (n,))
        w *= 2
    return v * np.float32(1.0 / math.sqrt(n))


def apply_rht_f32(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``apply_rht_np`` (``rht.py:51-57``): float32 ``hadamard(x * signs)``."""

    return hadamard_f32(np.asarray(x, dtype=np.float32) * np.asarray(signs, dtype=np.float32))


def apply_inverse_rht_f32(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """``apply_inverse_rht_np`` (``rht.py:60-66``): float32 ``hadamard(x) * signs``."""

    return hadamard_f32(x) * np.asarray(signs, dtype=np.float32)
