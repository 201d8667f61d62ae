"""Nearest-codeword encoders and the data-free RTN quantiser on the GPU.

- ``encode_e8p_rtn`` / ``encode_e8p_rtn_diagonal_hessian`` /
  ``encode_e8_1bit_rtn``: the E8P (uint16) and 8-bit E8 (uint8) nearest
  codeword of each 8-vector, optionally under a diagonal metric, through
  ``keep_vq_encode`` (the factored E8P search, ``src/keep/vq/e8.py:367-539``).
  The result is the exhaustive scan's: distances in double precision, ties to
  the lowest code (the reference's float32 search agrees wherever its rounding
  does not reorder near-ties).
- ``quantize_weight_rtn``: per (row, group) max-abs (or 99th percentile)
  scales over the codebook's largest magnitude, each vector divided by its
  scale and rounded to the nearest codeword (``src/keep/quant/rtn.py:253-318``);
  codes and fp16 scales stay on the device.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from keep_amd import _lib, ops

CODEWORD_DIM = 8


@dataclass
class QuantizedWeight:
    """Codes (uint8 / int16 holding uint16 bits) and fp16 scales on the device
    (``src/keep/quant/rtn.py:23-30``)."""

    codes: torch.Tensor
    scales: torch.Tensor
    codebook: np.ndarray
    group_size: int
    code_bits: int
    scale_estimator: str = "max_abs"


def _vectors(vectors, device=None) -> tuple[torch.Tensor, tuple]:
    t = vectors if isinstance(vectors, torch.Tensor) else torch.from_numpy(np.array(vectors, dtype=np.float32))
    if t.shape[-1] != CODEWORD_DIM:
        raise ValueError(f"vectors must have trailing dimension {CODEWORD_DIM}")
    dev = device or (t.device if t.is_cuda else torch.device("cuda", torch.cuda.current_device()))
    return t.to(device=dev, dtype=torch.float32).reshape(-1, CODEWORD_DIM).contiguous(), tuple(t.shape[:-1])


def _encode(flat: torch.Tensor, code_bits: int, diagonal=None, diag_mode: int = 0, scales=None, vps: int = 1):
    device = flat.device
    n = flat.shape[0]
    out = torch.empty(n, dtype=torch.int16 if code_bits == 16 else torch.uint8, device=device)
    table = ops._default_codebook(code_bits, device)
    _lib.call("keep_vq_encode", flat.data_ptr(), n, code_bits, ops._ptr(diagonal), diag_mode, table.data_ptr(),
              ops._ptr(scales), vps, out.data_ptr(), ops._stream(device))
    return out


def encode_e8p_rtn(vectors, *, chunk_size: int = 8192) -> torch.Tensor:
    """Nearest E8P codeword of each vector (``e8.py:367-445``): int16 codes
    holding the uint16 bits, shape ``vectors.shape[:-1]``."""

    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    flat, lead = _vectors(vectors)
    return _encode(flat, 16).reshape(lead)


def encode_e8p_rtn_diagonal_hessian(vectors, diagonal, *, chunk_size: int = 65536) -> torch.Tensor:
    """Nearest E8P codeword under ``sum_i w_i (v_i - c_i)^2`` with one shared
    diagonal ``[8]`` or one per vector (``e8.py:455-539``)."""

    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    flat, lead = _vectors(vectors)
    w = diagonal if isinstance(diagonal, torch.Tensor) else torch.from_numpy(np.array(diagonal, np.float32))
    w = w.to(device=flat.device, dtype=torch.float32).contiguous()
    if w.ndim == 1:
        if tuple(w.shape) != (CODEWORD_DIM,) or not bool(torch.isfinite(w).all()) or bool((w < 0).any()) \
                or not bool((w > 0).any()):
            raise ValueError("diagonal must be finite, non-negative, shape (8,), and nonzero")
        mode = 1
    else:
        w = w.reshape(-1, CODEWORD_DIM) if w.numel() == flat.numel() else w
        if tuple(w.shape) != tuple(flat.shape) or not bool(torch.isfinite(w).all()) or bool((w < 0).any()) \
                or not bool((w > 0).any(dim=1).all()):
            raise ValueError("per-row diagonal must be finite, non-negative, shape (N, 8), and nonzero per row")
        mode = 2
    return _encode(flat, 16, w, mode).reshape(lead)


def encode_e8_1bit_rtn(vectors) -> torch.Tensor:
    """Nearest entry of the 256-entry 8-bit E8 table (``e8.py:283-287``): uint8."""

    flat, lead = _vectors(vectors)
    return _encode(flat, 8).reshape(lead)


def codebook_max_abs(code_bits: int) -> float:
    """Largest |value| of the full codebook, the scale divisor (``rtn.py:48-54,260``)."""

    if code_bits == 16:
        half = np.stack([((ops.e8p_packed_abs_grid().astype(np.int64) >> (4 * d)) & 0xF) - 8 for d in range(8)], -1)
        return float(np.float32(np.abs(half).max() * 0.5) + np.float32(0.25))
    half = np.stack([((ops.e8_1bit_packed().astype(np.int64) >> (4 * d)) & 0xF) - 8 for d in range(8)], -1)
    return float(np.float32(np.abs(half).max() * 0.5))


def quantize_weight_rtn(weight, *, group_size: int = 512, code_bits: int = 8, codeword_chunk_size: int = 65536,
                        scale_estimator: str = "max_abs") -> QuantizedWeight:
    """Data-free RTN of a dense ``[out, in]`` weight (``rtn.py:270-318``): per
    (row, group) scale = max |w| (or the 99th percentile of |w|) over the
    codebook's largest magnitude; a zero scale divides by 1 and is stored as 0."""

    if code_bits not in (8, 16):
        raise ValueError("code_bits must be 8 or 16")
    w = weight if isinstance(weight, torch.Tensor) else torch.from_numpy(np.asarray(weight, dtype=np.float32))
    device = w.device if w.is_cuda else torch.device("cuda", torch.cuda.current_device())
    w = w.to(device=device, dtype=torch.float32).contiguous()
    if w.ndim != 2:
        raise ValueError(f"weight must be 2D [out, in], found shape {tuple(w.shape)}")
    if w.shape[1] % CODEWORD_DIM != 0:
        raise ValueError("weight input dimension must be divisible by 8")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    if w.shape[1] % group_size != 0:
        raise ValueError("weight input dimension must be divisible by group_size")
    if group_size % CODEWORD_DIM != 0:
        raise ValueError("group_size must be divisible by 8")
    if scale_estimator not in ("max_abs", "percentile_99"):
        raise ValueError(f"unknown scale_estimator {scale_estimator!r}")
    out_dim, in_dim = w.shape
    groups = in_dim // group_size
    divisor = codebook_max_abs(code_bits)
    if scale_estimator == "max_abs":
        scales = torch.empty((out_dim, groups), dtype=torch.float32, device=device)
        _lib.call("keep_group_absmax", w.data_ptr(), out_dim * groups, group_size, divisor, scales.data_ptr(),
                  ops._stream(device))
    else:
        q = torch.quantile(w.abs().reshape(out_dim, groups, group_size), 0.99, dim=-1)
        scales = (q.double() / divisor).float()
    safe = torch.where(scales > 0, scales, torch.ones_like(scales)).contiguous()
    codes = _encode(w.reshape(-1, CODEWORD_DIM), code_bits, scales=safe, vps=group_size // CODEWORD_DIM)
    table = ops.e8_1bit_packed() if code_bits == 8 else ops.e8p_packed_abs_grid()
    return QuantizedWeight(codes=codes.reshape(out_dim, in_dim // CODEWORD_DIM), scales=scales.half(),
                           codebook=table, group_size=group_size, code_bits=code_bits,
                           scale_estimator=scale_estimator)
