"""Random-sign Walsh-Hadamard transform of activations on the GPU.

``x -> FWHT(x * signs) / sqrt(n)`` over the last axis (orthonormal Sylvester
order), the activation-side RHT of the reference (``src/keep/quant/rht.py:51-91``,
applied in ``src/ramp/nn/switch_linear.py:320-322``), and its inverse
``x -> FWHT(x) / sqrt(n) * signs`` (``rht.py:60-66``). Computed by the HIP
kernel behind ``keep_rht``: float32 butterflies in the reference's stage order,
so a float32 result is bit-identical to the reference's numpy path; the
result is returned in the input dtype unless ``out_dtype`` says otherwise.
Rows of 16 to 8192 values are served; other widths raise ``ValueError``.

Deliberate deviation: for fp16 / bf16 ``x`` the reference's MLX path
(``apply_rht_mx``, ``rht.py:84-91``) runs the butterflies and the scale in
``x``'s dtype, rounding at every stage; here they run in float32 and the
result is rounded once, so it is the float32 result rounded to ``x``'s dtype
(closer to the exact transform, not bit-identical to the MLX one). Signs are
checked to be +-1, as ``_validate_signs_np`` (``rht.py:15-21``) checks them.
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


def check_signs(signs) -> None:
    """``ValueError`` unless every sign is -1 or 1 (``_validate_signs_np``,
    ``rht.py:15-21``). A device tensor is checked with one host sync."""

    t = signs if isinstance(signs, torch.Tensor) else torch.as_tensor(np.asarray(signs))
    if not bool(((t == 1) | (t == -1)).all()):
        raise ValueError("rht_signs values must be -1 or 1")


def _run(x: torch.Tensor, signs, inverse: bool, out_dtype: torch.dtype | None,
         validate_signs: bool = True) -> torch.Tensor:
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
        if validate_signs:
            check_signs(s)
    xc = x.contiguous()
    rows = xc.numel() // n
    out = torch.empty(x.shape, dtype=od, device=x.device)
    _lib.call("keep_rht", xc.data_ptr(), _DT[xc.dtype], None if s is None else s.data_ptr(), int(inverse), rows, n,
              out.data_ptr(), _DT[od], _stream(x.device))
    return out


def fwht(x: torch.Tensor, *, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Orthonormal FWHT over the last axis (``_hadamard_np``, ``rht.py:34-48``)."""

    return _run(x, None, False, out_dtype)


def apply_rht(x: torch.Tensor, signs, *, out_dtype: torch.dtype | None = None,
              validate_signs: bool = True) -> torch.Tensor:
    """``FWHT(x * signs) / sqrt(n)`` (``apply_rht_np`` ``rht.py:51-57``, ``apply_rht_mx`` ``:84-91``).
    ``validate_signs=False`` skips the +-1 check (a host sync) for signs already checked."""

    return _run(x, signs, False, out_dtype, validate_signs)


def apply_inverse_rht(x: torch.Tensor, signs, *, out_dtype: torch.dtype | None = None,
                      validate_signs: bool = True) -> torch.Tensor:
    """``FWHT(x) / sqrt(n) * signs`` (``apply_inverse_rht_np`` ``rht.py:60-66``)."""

    return _run(x, signs, True, out_dtype, validate_signs)
