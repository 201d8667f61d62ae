"""Random-sign Walsh-Hadamard transform of activations on the GPU.

``x -> FWHT(x * signs) / sqrt(n)`` over the last axis (orthonormal Sylvester
order), the activation-side RHT of the reference (``src/keep/quant/rht.py:51-91``,
applied in ``src/ramp/nn/switch_linear.py:320-322``), and its inverse
``x -> FWHT(x) / sqrt(n) * signs`` (``rht.py:60-66``). Computed by the HIP
kernel behind ``keep_rht``: float32 butterflies in the reference's stage order,
so a float32 result is bit-identical to the reference's numpy path; the
result is returned in the input dtype unless ``out_dtype`` says otherwise.
Rows of 16 to 8192 values are served; other widths raise ``ValueError``.
"""

from __future__ import annotations

import hashlib

import numpy as np
import torch

from keep_amd import _lib


def deterministic_rht_signs(dim: int, *, seed) -> np.ndarray:
    """+-1 int8 signs from ``shake_256(str(seed))`` little-endian bits, 0 -> -1
    (reference ``rht.py:24-31``)."""

    if dim <= 0 or dim & (dim - 1):
        raise ValueError("RHT dimension must be a positive power of two")
    raw = np.frombuffer(hashlib.shake_256(str(seed).encode("utf-8")).digest((dim + 7) // 8), dtype=np.uint8)
    bits = np.unpackbits(raw, bitorder="little")[:dim]
    return np.where(bits == 0, np.int8(-1), np.int8(1))


def _check_dim(n: int) -> None:
    if n <= 0 or n & (n - 1):
        raise ValueError("RHT dimension must be a positive power of two")
    if n < 16 or n > 8192:
        raise ValueError(f"keep_rht serves 16 <= n <= 8192, found {n}")


def _run(x: torch.Tensor, signs, inverse: bool, out_dtype: torch.dtype | None) -> torch.Tensor:
    from keep_amd.ops import _DT, _stream

    n = x.shape[-1]
    _check_dim(n)
    if not x.is_cuda:
        raise ValueError("apply_rht needs a device tensor")
    if x.dtype not in _DT:
        x = x.float()
    od = out_dtype or x.dtype
    if od not in _DT:
        raise ValueError(f"unsupported output dtype {od}")
    s = None
    if signs is not None:
        s = torch.as_tensor(signs, device=x.device).to(torch.float32).contiguous()
        if s.shape != (n,):
            raise ValueError(f"rht_signs must have shape ({n},), found {tuple(s.shape)}")
    xc = x.contiguous()
    rows = xc.numel() // n
    out = torch.empty(x.shape, dtype=od, device=x.device)
    _lib.call("keep_rht", xc.data_ptr(), _DT[xc.dtype], None if s is None else s.data_ptr(), int(inverse), rows, n,
              out.data_ptr(), _DT[od], _stream(x.device))
    return out


def fwht(x: torch.Tensor, *, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Orthonormal FWHT over the last axis (``_hadamard_np``, ``rht.py:34-48``)."""

    return _run(x, None, False, out_dtype)


def apply_rht(x: torch.Tensor, signs, *, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``FWHT(x * signs) / sqrt(n)`` (``apply_rht_np`` ``rht.py:51-57``, ``apply_rht_mx`` ``:84-91``)."""

    return _run(x, signs, False, out_dtype)


def apply_inverse_rht(x: torch.Tensor, signs, *, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``FWHT(x) / sqrt(n) * signs`` (``apply_inverse_rht_np`` ``rht.py:60-66``)."""

    return _run(x, signs, True, out_dtype)
