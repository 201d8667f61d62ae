"""Random-sign Walsh-Hadamard transform of activations on the GPU.

``x -> FWHT(x * signs) / sqrt(n)`` over the last axis (orthonormal Sylvester
order), the activation-side RHT of the reference (``src/keep/quant/rht.py:51-91``,
applied in ``src/ramp/nn/switch_linear.py:320-322``). Computed in float32 with
torch ops on the device and returned in the input dtype.
"""

from __future__ import annotations

import hashlib
import math

import numpy as np
import torch


def deterministic_rht_signs(dim: int, *, seed) -> np.ndarray:
    """+-1 int8 signs from ``shake_256(str(seed))`` little-endian bits, 0 -> -1
    (reference ``rht.py:24-31``)."""

    if dim <= 0 or dim & (dim - 1):
        raise ValueError("RHT dimension must be a positive power of two")
    raw = np.frombuffer(hashlib.shake_256(str(seed).encode("utf-8")).digest((dim + 7) // 8), dtype=np.uint8)
    bits = np.unpackbits(raw, bitorder="little")[:dim]
    return np.where(bits == 0, np.int8(-1), np.int8(1))


def fwht(x: torch.Tensor) -> torch.Tensor:
    n = x.shape[-1]
    if n <= 0 or n & (n - 1):
        raise ValueError("RHT dimension must be a positive power of two")
    lead = x.shape[:-1]
    v = x.reshape(-1, n)
    h = 1
    while h < n:
        v = v.reshape(-1, n // (2 * h), 2, h)
        a, b = v[:, :, 0, :], v[:, :, 1, :]
        v = torch.stack((a + b, a - b), dim=2).reshape(-1, n)
        h *= 2
    return (v * (1.0 / math.sqrt(n))).reshape(*lead, n)


def apply_rht(x: torch.Tensor, signs) -> torch.Tensor:
    s = torch.as_tensor(signs, device=x.device).to(torch.float32)
    if s.shape != (x.shape[-1],):
        raise ValueError(f"rht_signs must have shape ({x.shape[-1]},), found {tuple(s.shape)}")
    return fwht(x.float() * s).to(x.dtype)
