"""The steps either side of the routed experts -- CPU oracle (test
infrastructure only; see ``oracle/__init__.py``).

- ``rmsnorm``: ``gamma * x / sqrt(mean(x^2) + eps)`` in fp32 math, rounded once
  to the row dtype (the block's ``ffn_norm``,
  ``src/ramp/models/deepseek_v4_flash_adapter.py:1794,1806``).
- ``e4m3_round`` / ``act_quant``: block-wise FP8 e4m3 fake quantisation of the
  normed activations (``scripts/runpod/v41_reap/torch_kernel.py:25-53``: amax
  per block clamped to 1e-4, scale amax / 448, optionally rounded up to a
  power of two, values clamped to +-448, rounded to e4m3 and scaled back into
  the row dtype), the expert input of the serving step
  (``scripts/v41_build/omlx_lattice.py:332,357``).
- ``shared_combine``: the routed sum plus the shared expert, plus the residual,
  rounded to the output dtype (``deepseek_v4_flash_adapter.py:1784``; the
  serving step adds the fp32 routed sum inside the shared down projection and
  rounds to bf16, ``omlx_lattice.py:374-388``).

Pins (``tests/test_oracle_block.py``): ``e4m3_round`` against torch's own
float8_e4m3fn conversion over every bf16 value in range and every tie between
neighbouring e4m3 values; ``pow2_ceil`` against ``2 ** ceil(log2 v)``;
``rmsnorm`` against its closed form on constant rows and its scale invariance;
``act_quant`` against the e4m3 grid (every output / scale is an e4m3 value
within half a step of the input) and idempotence under power-of-two scales.
"""

from __future__ import annotations

import numpy as np

from oracle.ops import round_bf16

FP8_MAX = 448.0


def round_to(a, dtype: str) -> np.ndarray:
    """Round fp32 values to ``dtype`` ("bfloat16", "float16", "float32"), returned as float32."""

    a = np.asarray(a, dtype=np.float32)
    if dtype == "bfloat16":
        return round_bf16(a).astype(np.float32)
    if dtype == "float16":
        return a.astype(np.float16).astype(np.float32)
    return a


def rmsnorm(x, gamma=None, eps: float = 1e-6, dtype: str = "float32") -> np.ndarray:
    """``round_dtype(gamma * (x * (1 / sqrt(mean(x^2) + eps))))`` per row, fp32 math."""

    x = np.asarray(x, dtype=np.float32)
    ms = (x.astype(np.float64) ** 2).mean(-1, keepdims=True).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32)
    y = x * inv
    if gamma is not None:
        y = np.asarray(gamma, dtype=np.float32) * y
    return round_to(y, dtype)


def e4m3_round(v) -> np.ndarray:
    """Nearest FP8 e4m3fn value of fp32 ``v`` (|v| <= 448), ties to even: three
    mantissa bits at |v| >= 2^-6, a fixed step of 2^-9 below."""

    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v)
    b = a.view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFFF + ((b >> 20) & 1)) & 0xFFF00000
    normal = b.astype(np.uint32).view(np.float32)
    sub = (np.rint(a.astype(np.float64) * 512.0) / 512.0).astype(np.float32)
    return np.copysign(np.where(a >= np.float32(2.0 ** -6), normal, sub), v).astype(np.float32)


def pow2_ceil(v) -> np.ndarray:
    """``2 ** ceil(log2 v)`` of positive normal fp32 values, by their exponent bits."""

    b = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.int64)
    e = ((b >> 23) & 0xFF) - 127 + ((b & 0x7FFFFF) != 0)
    return ((e + 127) << 23).astype(np.uint32).view(np.float32)


def act_quant(y, block: int = 128, pow2: bool = False, dtype: str = "float32") -> np.ndarray:
    """Block-wise FP8 e4m3 fake quantisation of rows ``y`` (fp32 values of ``dtype``)."""

    y = np.asarray(y, dtype=np.float32)
    yb = y.reshape(y.shape[:-1] + (-1, block))
    amax = np.maximum(np.abs(yb).max(-1), np.float32(1e-4))
    s = (amax * np.float32(1.0 / FP8_MAX)).astype(np.float32)
    if pow2:
        s = pow2_ceil(s)
    q = e4m3_round(np.clip(yb / s[..., None], -FP8_MAX, FP8_MAX).astype(np.float32))
    return round_to(q * s[..., None], dtype).reshape(y.shape)


def norm_quant(x, gamma=None, eps: float = 1e-6, *, block: int = 128, pow2: bool = False,
               dtype: str = "float32") -> tuple[np.ndarray, np.ndarray]:
    """``(normed, quantised)`` rows, both fp32 values of ``dtype`` (block 0: no quantisation)."""

    y = rmsnorm(x, gamma, eps, dtype)
    return y, (act_quant(y, block, pow2, dtype) if block else y)


def shared_combine(routed, shared=None, residual=None, dtype: str = "bfloat16") -> np.ndarray:
    """``round_dtype(residual + (routed + shared))`` with fp32 sums, in that order."""

    acc = np.asarray(routed, dtype=np.float32)
    if shared is not None:
        acc = (acc + np.asarray(shared, dtype=np.float32)).astype(np.float32)
    if residual is not None:
        acc = (np.asarray(residual, dtype=np.float32) + acc).astype(np.float32)
    return round_to(acc, dtype)
