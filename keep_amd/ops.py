"""Routed VQ operators over torch device tensors, drop-in for the reference's
MLX operators, running the gfx950 HIP kernels of ``libkeep_amd.so``.

Signatures, argument meaning and error behaviour follow the reference
(``src/ramp/kernels/vq_qmv.py``, ``vq_qmm.py``, ``e8p_m1.py``,
``e8p_nested_m1.py`` and ``src/ramp/ops/vq_switch.py``); arrays are torch
tensors on a ROCm device instead of ``mx.array``. Differences, each deliberate:

- ``implementation``: ``"hip"`` (default) and ``"metal"`` (accepted as an
  alias so existing callers keep working) both run the HIP kernels.
  ``"reference"`` raises ``ValueError``: the dense CPU oracle is test
  infrastructure here, never a product path.
- ``codebook_duplication`` / ``rows_per_simdgroup`` / ``simdgroups`` /
  ``rows_per_threadgroup`` are validated as in the reference and otherwise
  ignored: the LDS codebook and the wave-per-rows layout are fixed by the
  gfx950 kernels.
- Contract violations raise ``ValueError`` before any launch, as in the
  reference (``vq_switch.py:491-544``); a missing HIP library raises
  ``RuntimeError``. Index ranges are checked on the host only with
  ``validate_indices=True`` (it syncs); a route index out of range on the
  device yields a NaN output row, never a fault.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from typing import Any, Iterator, Literal

import numpy as np
import torch

from keep_amd import _lib

CODEWORD_DIM = 8
NO_RESIDUAL = 0xFFFFFFFF
# Route count from which E8P calls go to the MFMA grouped GEMM (prefill);
# below it the wave-per-rows mat-vec serves every route directly.
GEMM_ROUTE_THRESHOLD = 128
GEMM_ROUTE_TILE = 64
_VERIFY_DEFAULT_M_ROWS = 4
VERIFY_MROWS_VALUES = (1, 2, 3, 4, 8)

_TRACE: ContextVar[list[dict[str, Any]] | None] = ContextVar("keep_amd_gather_trace", default=None)


@contextmanager
def trace_gather_vqmm_calls() -> Iterator[list[dict[str, Any]]]:
    """Record every routed dispatch (reference ``vq_switch.py:70-84``)."""

    records: list[dict[str, Any]] = []
    token = _TRACE.set(records)
    try:
        yield records
    finally:
        _TRACE.reset(token)


def _trace(**rec) -> None:
    t = _TRACE.get()
    if t is not None:
        t.append(rec)


# --------------------------------------------------------------------------- codebooks


_HOST_TABLES: dict[int, np.ndarray] = {}
_DEVICE_TABLES: dict[tuple[int, str], torch.Tensor] = {}


def e8p_packed_abs_grid() -> np.ndarray:
    """``uint32[256]`` E8P packed abs table, built by the library's closed form."""

    if 16 not in _HOST_TABLES:
        out = (_lib.c_uint32 * 256)()
        _lib.call("keep_e8p_packed_abs_grid", out)
        _HOST_TABLES[16] = np.frombuffer(out, dtype=np.uint32).copy()
    return _HOST_TABLES[16].copy()


def e8_1bit_packed() -> np.ndarray:
    """``uint32[256]`` packed 8-bit E8 residual table."""

    if 8 not in _HOST_TABLES:
        out = (_lib.c_uint32 * 256)()
        _lib.call("keep_e8_1bit_packed", out)
        _HOST_TABLES[8] = np.frombuffer(out, dtype=np.uint32).copy()
    return _HOST_TABLES[8].copy()


def _default_codebook(code_bits: int, device: torch.device) -> torch.Tensor:
    key = (code_bits, str(device))
    if key not in _DEVICE_TABLES:
        host = e8p_packed_abs_grid() if code_bits == 16 else e8_1bit_packed()
        _DEVICE_TABLES[key] = torch.from_numpy(host.view(np.int32)).to(device)
    return _DEVICE_TABLES[key]


_PREPARED: dict[tuple[int, str], tuple[torch.Tensor, torch.Tensor]] = {}


def prepared_table(codebook: torch.Tensor) -> torch.Tensor:
    """The prepared E8P table of ``codebook`` for the matrix-core kernels
    (``keep_e8p_prepare``: T and M of the int8 decode, a check word and the
    64 KiB LDS image, ``keep_e8p_prepared_bytes()`` bytes), cached per codebook tensor."""

    key = (codebook.data_ptr(), str(codebook.device))
    hit = _PREPARED.get(key)
    if hit is not None and hit[0] is codebook:
        return hit[1]
    nbytes = _lib.load().keep_e8p_prepared_bytes()
    out = torch.empty(nbytes, dtype=torch.uint8, device=codebook.device)
    _lib.call("keep_e8p_prepare", codebook.data_ptr(), out.data_ptr(), _stream(codebook.device))
    _PREPARED[key] = (codebook, out)
    return out


def half2_pairs(grid: np.ndarray) -> np.ndarray:
    """``[256, 8]`` codebook exact in fp16 -> ``uint32[256, 4]`` (entry k = fp16
    bits of dim 2k | dim 2k+1 << 16), as ``e8p_nested_m1.half2_pairs``."""

    h = np.asarray(grid).astype(np.float16)
    if h.shape != (256, 8) or not np.array_equal(h.astype(np.float64), np.asarray(grid, dtype=np.float64)):
        raise ValueError("codebook must be [256, 8] and exact in float16")
    bits = h.view(np.uint16).astype(np.uint32)
    return np.ascontiguousarray(bits[:, 0::2] | (bits[:, 1::2] << 16))


def e8_1bit_half2_table() -> np.ndarray:
    """The 8-bit E8 table as ``half2_pairs`` (the nested residual's table)."""

    t = e8_1bit_packed().astype(np.int64)
    grid = np.stack([((t >> (4 * d)) & 0xF) - 8 for d in range(8)], axis=-1).astype(np.float64) * 0.5
    return half2_pairs(grid)


# --------------------------------------------------------------------------- tensor plumbing

_DT = {torch.float32: _lib.KEEP_F32, torch.float16: _lib.KEEP_F16, torch.bfloat16: _lib.KEEP_BF16}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"{what} dtype must be float32, float16 or bfloat16, found {t.dtype}") from None


def output_dtype(x_dtype: torch.dtype) -> torch.dtype:
    """Output dtype follows x (reference ``vq_qmv.py:40-46``)."""

    return x_dtype if x_dtype in (torch.float16, torch.bfloat16) else torch.float32


def _device_of(*ts) -> torch.device:
    for t in ts:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("keep_amd operators need a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def _to_dev(a, device: torch.device, dtype: torch.dtype | None = None) -> torch.Tensor:
    if isinstance(a, np.ndarray):
        if a.dtype == np.uint16:
            a = a.view(np.int16)
        elif a.dtype == np.uint32:
            a = a.view(np.int32)
        a = torch.from_numpy(np.ascontiguousarray(a))
    elif not isinstance(a, torch.Tensor):
        a = torch.as_tensor(a)
    if a.dtype == torch.uint16:
        a = a.view(torch.int16)
    elif a.dtype == torch.uint32:
        a = a.view(torch.int32)
    if dtype is not None and a.dtype != dtype:
        a = a.to(dtype)
    return a.to(device).contiguous()


def _codes_tensor(codes, code_bits: int, device) -> torch.Tensor:
    t = codes if isinstance(codes, torch.Tensor) else None
    name = str(t.dtype if t is not None else np.asarray(codes).dtype)
    want = ("uint16", "int16") if code_bits == 16 else ("uint8", "int8")
    if name.rsplit(".", 1)[-1] not in want:
        raise ValueError(f"codes dtype must be {'uint16' if code_bits == 16 else 'uint8'}, found {name}")
    out = _to_dev(codes, device)
    return out.view(torch.int16) if code_bits == 16 and out.dtype == torch.uint16 else out


def _code_bits_of(codes) -> int:
    """8 for uint8/int8 codes (8-bit E8), 16 for uint16/int16 (E8P)."""

    name = str(codes.dtype if isinstance(codes, torch.Tensor) else np.asarray(codes).dtype).rsplit(".", 1)[-1]
    if name in ("uint8", "int8"):
        return 8
    if name in ("uint16", "int16"):
        return 16
    raise ValueError(f"codes dtype must be uint8 (8-bit E8) or uint16 (E8P), found {name}")


def _codebook_tensor(codebook, code_bits: int, device) -> torch.Tensor:
    if codebook is None:
        return _default_codebook(code_bits, device)
    name = str(codebook.dtype).rsplit(".", 1)[-1]
    if name not in ("uint32", "int32"):
        raise ValueError(f"codebook dtype must be uint32, found {codebook.dtype}")
    if tuple(codebook.shape) != (256,):
        raise ValueError(f"codebook must have shape (256,), found {tuple(codebook.shape)}")
    return _to_dev(codebook, device)


def _index_tensor(ix, device) -> torch.Tensor:
    t = ix if isinstance(ix, torch.Tensor) else torch.as_tensor(np.asarray(ix))
    if t.dtype.is_floating_point or t.dtype == torch.bool:
        raise ValueError(f"indices must use an integer dtype, found {t.dtype}")
    return _to_dev(t, device, torch.int32)


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_impl(implementation: str) -> None:
    if implementation == "reference":
        raise ValueError("implementation='reference' is the CPU oracle; it lives in the test suite (oracle/), "
                         "not in the product path")
    if implementation not in ("hip", "metal", "auto"):
        raise ValueError("implementation must be 'hip' (or its alias 'metal')")


def _check_dup(codebook_duplication: int) -> None:
    if codebook_duplication not in (1, 4, 8):
        raise ValueError("codebook_duplication must be 1, 4, or 8")


def _validate_dims(input_dims: int, output_dims: int, group_size: int, code_bits: int) -> None:
    if code_bits not in (8, 16):
        raise ValueError("code_bits must be 8 or 16")
    if input_dims <= 0 or output_dims <= 0:
        raise ValueError("input_dims and output_dims must be positive")
    if input_dims % CODEWORD_DIM != 0:
        raise ValueError("input_dims must be divisible by 8")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    if input_dims % group_size != 0:
        raise ValueError("input_dims must be divisible by group_size")
    if group_size % CODEWORD_DIM != 0:
        raise ValueError("group_size must be divisible by 8 on the HIP kernels")


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


# --------------------------------------------------------------------------- raw launchers


def routed_matvec(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor, codebook: torch.Tensor,
                  rhs: torch.Tensor | None, *, lhs: torch.Tensor | None = None, x_div: int = 1, input_dims: int,
                  output_dims: int, group_size: int, code_bits: int = 16, residual=None, hot_of_slot=None,
                  out_dtype: torch.dtype | None = None, routes: int | None = None) -> torch.Tensor:
    """``out[r] = W[rhs[r]] . x[lhs[r] or r // x_div]`` -> ``[routes, N]`` (``keep_vq_matvec``).
    ``rhs=None`` (one matrix, ``codes [1, N, K/8]``): every one of ``routes`` routes reads it.

    ``residual`` = ``(res_codes uint8 [H, N, K/8], res_scales [H, N, G'], res_table [256, 4])``
    with ``hot_of_slot`` ``uint32 [E]``.
    """

    device = x.device
    if rhs is not None:
        routes = rhs.numel()
    elif routes is None or codes.shape[0] != 1:
        raise ValueError("rhs=None needs routes and a single matrix")
    od = out_dtype or output_dtype(x.dtype)
    out = torch.empty((routes, output_dims), dtype=od, device=device)
    if routes == 0:
        return out
    E = codes.shape[0]
    rc = rs = rt = hot = None
    rgs = 0
    nhot = 0
    if residual is not None:
        rc, rs, rt = residual
        rgs = input_dims // rs.shape[-1]
        hot = hot_of_slot
        nhot = rc.shape[0]
        if rs.dtype != scales.dtype:
            rs = rs.to(scales.dtype)
    _lib.call("keep_vq_matvec", x.data_ptr(), _dtype_code(x, "x"), x.shape[0], codes.data_ptr(), code_bits,
              scales.data_ptr(), _dtype_code(scales, "scales"), codebook.data_ptr(), _ptr(rhs), _ptr(lhs),
              routes, x_div, E, output_dims, input_dims, group_size, _ptr(rc), _ptr(rs), rgs, _ptr(rt), _ptr(hot),
              nhot, out.data_ptr(), _DT[od], _stream(device))
    return out


def route_plan(rhs: torch.Tensor, num_experts: int, tile: int):
    """Device route plan (``keep_route_plan``): ``(order, inverse, counts, offsets,
    tile_expert, tile_offset, tile_count, n_tiles)``; ``n_tiles`` is a 1-element
    device tensor (no host sync)."""

    device = rhs.device
    R = rhs.numel()
    max_tiles = (R + tile - 1) // tile + num_experts
    i32 = dict(dtype=torch.int32, device=device)
    order = torch.empty(R, **i32)
    inverse = torch.empty(R, **i32)
    counts = torch.empty(num_experts, **i32)
    offsets = torch.empty(num_experts, **i32)
    te = torch.empty(max_tiles, **i32)
    to = torch.empty(max_tiles, **i32)
    tc = torch.empty(max_tiles, **i32)
    nt = torch.empty(1, **i32)
    _lib.call("keep_route_plan", _ptr(rhs) if R else None, R, num_experts, tile, _ptr(order) if R else None,
              _ptr(inverse) if R else None, counts.data_ptr(), offsets.data_ptr(), te.data_ptr(), to.data_ptr(),
              tc.data_ptr(), max_tiles, nt.data_ptr(), _stream(device))
    return order, inverse, counts, offsets, te, to, tc, nt


def _q8_workspace(rows: int, K: int, device: torch.device) -> torch.Tensor:
    n = int(_lib.load().keep_vq_grouped_gemm_q8_workspace_bytes(rows, K))
    return torch.empty((n,), dtype=torch.uint8, device=device)


def grouped_gemm(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor, codebook: torch.Tensor,
                 tile_descriptors, *, lhs: torch.Tensor | None, routes: int, input_dims: int, output_dims: int,
                 group_size: int, out_dtype: torch.dtype | None = None,
                 out_index: torch.Tensor | None = None) -> torch.Tensor:
    """``keep_vq_grouped_gemm_q8``: sorted-route GEMM on the fp16 matrix cores ->
    ``[routes, N]``, row ``p`` in sorted order, or row ``out_index[p]`` when
    ``out_index`` is given (the scatter back to route order folded in)."""

    device = x.device
    od = out_dtype or output_dtype(x.dtype)
    out = torch.empty((routes, output_dims), dtype=od, device=device)
    if routes == 0:
        return out
    te, to, tc = tile_descriptors
    xc = x.contiguous()
    ws = _q8_workspace(xc.shape[0], input_dims, device)
    prep = prepared_table(codebook)
    _lib.call("keep_vq_grouped_gemm_q8", xc.data_ptr(), _dtype_code(xc, "x"), xc.shape[0], _ptr(lhs),
              _ptr(out_index), codes.data_ptr(), 16, scales.data_ptr(), _dtype_code(scales, "scales"), prep.data_ptr(),
              te.data_ptr(), to.data_ptr(), tc.data_ptr(), te.numel(), routes, codes.shape[0], output_dims,
              input_dims, group_size, ws.data_ptr(), ws.numel(), out.data_ptr(), _DT[od], _stream(device))
    return out


def grouped_residual_add(out: torch.Tensor, x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
                         tile_descriptors, *, lhs: torch.Tensor | None, out_index: torch.Tensor | None, routes: int,
                         input_dims: int, output_dims: int, group_size: int,
                         table: torch.Tensor | None = None) -> torch.Tensor:
    """``keep_vq_grouped_gemm_q8`` on the nested tier's 8-bit E8 residual:
    ``out[out_index[p]] += R[hot row of tile] . x[lhs[p]]`` over tiles of routes
    grouped by residual row (``route_plan`` over the routes' hot rows). ``out``
    is fp32 ``[*, N]``; ``table`` is the packed 8-bit E8 table (default one)."""

    if out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("the residual is added into a contiguous float32 output")
    if routes == 0:
        return out
    device = x.device
    te, to, tc = tile_descriptors
    xc = x.contiguous()
    ws = _q8_workspace(xc.shape[0], input_dims, device)
    tab = _to_dev(e8_1bit_packed().view(np.int32), device) if table is None else table
    _lib.call("keep_vq_grouped_gemm_q8", xc.data_ptr(), _dtype_code(xc, "x"), xc.shape[0], _ptr(lhs),
              _ptr(out_index), codes.data_ptr(), 8, scales.data_ptr(), _dtype_code(scales, "scales"), tab.data_ptr(),
              te.data_ptr(), to.data_ptr(), tc.data_ptr(), te.numel(), routes, codes.shape[0], output_dims,
              input_dims, group_size, ws.data_ptr(), ws.numel(), out.data_ptr(), _DT[torch.float32],
              _stream(device))
    return out


def grouped_swiglu(x: torch.Tensor, gate_codes: torch.Tensor, gate_scales: torch.Tensor, up_codes: torch.Tensor,
                   up_scales: torch.Tensor, codebook: torch.Tensor, tile_descriptors, *, lhs: torch.Tensor | None,
                   routes: int, input_dims: int, hidden_dims: int, group_size: int,
                   limit: float = 0.0) -> torch.Tensor:
    """``keep_vq_grouped_swiglu_q8``: gate and up of the same sorted-route tiles
    in one pass, SwiGLU in fp32 -> bf16 ``h [routes, I]`` in sorted order."""

    device = x.device
    h = torch.empty((routes, hidden_dims), dtype=torch.bfloat16, device=device)
    if routes == 0:
        return h
    if gate_scales.dtype != up_scales.dtype:
        raise ValueError("gate and up scales must share a dtype")
    te, to, tc = tile_descriptors
    xc = x.contiguous()
    ws = _q8_workspace(xc.shape[0], input_dims, device)
    prep = prepared_table(codebook)
    _lib.call("keep_vq_grouped_swiglu_q8", xc.data_ptr(), _dtype_code(xc, "x"), xc.shape[0], _ptr(lhs),
              gate_codes.data_ptr(), gate_scales.data_ptr(), up_codes.data_ptr(), up_scales.data_ptr(),
              _dtype_code(gate_scales, "scales"), prep.data_ptr(), te.data_ptr(), to.data_ptr(), tc.data_ptr(),
              te.numel(), routes, gate_codes.shape[0], hidden_dims, input_dims, group_size, float(limit),
              ws.data_ptr(), ws.numel(), h.data_ptr(), _stream(device))
    return h


def _nested_residual(res, name: str, n: int, k: int):
    codes, scales = res
    if codes.dtype != torch.uint8 or tuple(codes.shape[1:]) != (n, k // 8) or not codes.is_contiguous():
        raise ValueError(f"{name} residual codes must be contiguous uint8 [rows, {n}, {k // 8}]")
    if scales.ndim != 3 or tuple(scales.shape) != (codes.shape[0], n, 1) or not scales.is_contiguous():
        raise ValueError(f"{name} residual scales must be contiguous [rows, {n}, 1] (one scale per row)")
    return codes, scales


def grouped_swiglu_nested(x: torch.Tensor, gate_codes: torch.Tensor, gate_scales: torch.Tensor,
                          up_codes: torch.Tensor, up_scales: torch.Tensor, codebook: torch.Tensor, gate_res, up_res,
                          hot_row: torch.Tensor, res_table: torch.Tensor, tile_descriptors, *,
                          lhs: torch.Tensor | None, routes: int, input_dims: int, hidden_dims: int,
                          limit: float = 0.0) -> torch.Tensor:
    """``keep_vq_grouped_swiglu_nested_q8``: ``grouped_swiglu`` (per-row base
    scales) with the nested tier's 8-bit E8 residual of each hot expert added
    to gate and up before the SwiGLU (``omlx_lattice.py:172-186``). ``gate_res``
    / ``up_res`` = (uint8 codes ``[rows, I, H / 8]``, scales ``[rows, I, 1]``),
    ``hot_row`` int32 ``[E]`` (-1: none), ``res_table`` the packed E8 table."""

    device = x.device
    h = torch.empty((routes, hidden_dims), dtype=torch.bfloat16, device=device)
    if routes == 0:
        return h
    if gate_scales.dtype != up_scales.dtype:
        raise ValueError("gate and up scales must share a dtype")
    grc, grs = _nested_residual(gate_res, "gate", hidden_dims, input_dims)
    urc, urs = _nested_residual(up_res, "up", hidden_dims, input_dims)
    if grs.dtype != urs.dtype or grc.shape[0] != urc.shape[0]:
        raise ValueError("gate and up residuals must share their rows and scale dtype")
    te, to, tc = tile_descriptors
    xc = x.contiguous()
    ws = _q8_workspace(xc.shape[0], input_dims, device)
    prep = prepared_table(codebook)
    _lib.call("keep_vq_grouped_swiglu_nested_q8", xc.data_ptr(), _dtype_code(xc, "x"), xc.shape[0], _ptr(lhs),
              gate_codes.data_ptr(), gate_scales.data_ptr(), up_codes.data_ptr(), up_scales.data_ptr(),
              _dtype_code(gate_scales, "scales"), prep.data_ptr(), grc.data_ptr(), grs.data_ptr(), urc.data_ptr(),
              urs.data_ptr(), _dtype_code(grs, "residual scales"), hot_row.data_ptr(), grc.shape[0],
              res_table.data_ptr(), te.data_ptr(), to.data_ptr(), tc.data_ptr(), te.numel(), routes,
              gate_codes.shape[0], hidden_dims, input_dims, float(limit), ws.data_ptr(), ws.numel(), h.data_ptr(),
              _stream(device))
    return h


def grouped_gemm_nested(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor, codebook: torch.Tensor, res,
                        hot_row: torch.Tensor, res_table: torch.Tensor, tile_descriptors, *,
                        lhs: torch.Tensor | None, routes: int, input_dims: int, output_dims: int,
                        out_dtype: torch.dtype | None = None, out_index: torch.Tensor | None = None) -> torch.Tensor:
    """``keep_vq_grouped_gemm_nested_q8``: ``grouped_gemm`` (per-row base
    scales) plus the nested tier's residual of each hot expert, added before
    the store (row ``out_index[p]`` when given)."""

    device = x.device
    od = out_dtype or output_dtype(x.dtype)
    out = torch.empty((routes, output_dims), dtype=od, device=device)
    if routes == 0:
        return out
    rc, rs = _nested_residual(res, "down", output_dims, input_dims)
    te, to, tc = tile_descriptors
    xc = x.contiguous()
    ws = _q8_workspace(xc.shape[0], input_dims, device)
    prep = prepared_table(codebook)
    _lib.call("keep_vq_grouped_gemm_nested_q8", xc.data_ptr(), _dtype_code(xc, "x"), xc.shape[0], _ptr(lhs),
              _ptr(out_index), codes.data_ptr(), scales.data_ptr(), _dtype_code(scales, "scales"), prep.data_ptr(),
              rc.data_ptr(), rs.data_ptr(), _dtype_code(rs, "residual scales"), hot_row.data_ptr(), rc.shape[0],
              res_table.data_ptr(), te.data_ptr(), to.data_ptr(), tc.data_ptr(), te.numel(), routes, codes.shape[0],
              output_dims, input_dims, ws.data_ptr(), ws.numel(), out.data_ptr(), _DT[od], _stream(device))
    return out


def route_combine(y: torch.Tensor, weight: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``keep_route_combine``: ``sum_j w[t, j] * y[t, j, :]`` in fp32 for
    ``y [T, k, H]`` (``glm4_moe_adapter.py:367-372``)."""

    T, k, H = y.shape
    od = out_dtype or torch.float32
    yf = y.float().contiguous()
    wf = weight.reshape(T, k).float().contiguous()
    if H % 4:
        raise ValueError(f"route_combine needs H a multiple of 4, found {H}")
    out = torch.empty((T, H), dtype=od, device=y.device)
    _lib.call("keep_route_combine", yf.data_ptr(), wf.data_ptr(), T, k, H, out.data_ptr(), _DT[od], _stream(y.device))
    return out


def gemm_eligible(*, code_bits: int, x_dtype: torch.dtype, input_dims: int, group_size: int) -> bool:
    """Whether the grouped GEMM (fp16 matrix cores) serves this call (E8P, fp16/bf16/fp32
    activations, K and the scale group multiples of 128)."""

    return (code_bits == 16 and x_dtype in (torch.float16, torch.bfloat16, torch.float32) and input_dims % 128 == 0
            and group_size % 128 == 0)


# --------------------------------------------------------------------------- decode


def decode_e8p(codes, codebook=None) -> torch.Tensor:
    """E8P codewords -> float32 ``[..., 8]`` on the GPU, bit-exact with the
    reference ``decode_e8p`` (``src/keep/vq/e8.py:210-234``)."""

    device = _device_of(codes, codebook)
    c = _codes_tensor(codes, 16, device)
    cb = _codebook_tensor(codebook, 16, device)
    out = torch.empty(tuple(c.shape) + (8,), dtype=torch.float32, device=device)
    _lib.call("keep_e8p_decode", c.data_ptr(), c.numel(), cb.data_ptr(), None, 0, 1, 1, out.data_ptr(),
              _stream(device))
    return out


def decode_weight_matrix(codes, scales=None, *, code_bits: int = 8, codebook=None) -> torch.Tensor:
    """Dense float32 weights ``[..., 8*C]`` (reference ``e8.py:542-571``): 8-bit
    E8 codes (uint8, the reference's default) or E8P (uint16)."""

    if code_bits not in (8, 16):
        raise ValueError("code_bits must be 8 or 16")
    fn = "keep_e8p_decode" if code_bits == 16 else "keep_e8_1bit_decode"
    device = _device_of(codes, scales, codebook)
    c = _codes_tensor(codes, code_bits, device)
    cb = _codebook_tensor(codebook, code_bits, device)
    C = c.shape[-1]
    out = torch.empty(tuple(c.shape[:-1]) + (C * 8,), dtype=torch.float32, device=device)
    if scales is None:
        _lib.call(fn, c.data_ptr(), c.numel(), cb.data_ptr(), None, 0, 1, 1, out.data_ptr(), _stream(device))
        return out
    s = _to_dev(scales, device)
    G = s.shape[-1]
    if C % G:
        raise ValueError("codeword count must be divisible by scale count")
    if tuple(s.shape[:-1]) != tuple(c.shape[:-1]):
        raise ValueError(f"scales leading shape {tuple(s.shape[:-1])} must match codes {tuple(c.shape[:-1])}")
    _lib.call(fn, c.data_ptr(), c.numel(), cb.data_ptr(), s.data_ptr(), _dtype_code(s, "scales"), C, C // G,
              out.data_ptr(), _stream(device))
    return out


# --------------------------------------------------------------------------- vq_qmv / vq_qmm


def vq_qmv(x, codes, scales, codebook=None, *, in_dim: int, out_dim: int, group_size: int = 512,
           code_bits: Literal[8, 16] = 8, implementation: str = "hip",
           codebook_duplication: Literal[1, 4, 8] = 1) -> torch.Tensor:
    """Decode-quantized mat-vec ``W x`` (reference ``vq_qmv.py:163-232``)."""

    _check_impl(implementation)
    _validate_dims(in_dim, out_dim, group_size, code_bits)
    _check_dup(codebook_duplication)
    device = _device_of(x, codes, scales)
    xt = _to_dev(x, device)
    if tuple(xt.shape) != (in_dim,):
        raise ValueError(f"x must have shape ({in_dim},), found {tuple(xt.shape)}")
    c = _codes_tensor(codes, code_bits, device)
    s = _to_dev(scales, device)
    if tuple(c.shape) != (out_dim, in_dim // 8):
        raise ValueError(f"codes must have shape ({out_dim}, {in_dim // 8}), found {tuple(c.shape)}")
    if tuple(s.shape) != (out_dim, in_dim // group_size):
        raise ValueError(f"scales must have shape ({out_dim}, {in_dim // group_size}), found {tuple(s.shape)}")
    cb = _codebook_tensor(codebook, code_bits, device)
    y = routed_matvec(xt.reshape(1, in_dim), c.reshape(1, out_dim, -1), s.reshape(1, out_dim, -1), cb, None,
                      input_dims=in_dim, output_dims=out_dim, group_size=group_size, code_bits=code_bits, routes=1)
    return y.reshape(out_dim)


def vq_qmm(x, codes, scales, codebook=None, *, in_dim: int, out_dim: int, group_size: int = 512,
           code_bits: Literal[8, 16] = 8, implementation: str = "hip",
           codebook_duplication: Literal[1, 4, 8] = 1) -> torch.Tensor:
    """``X W^T`` for ``x [M, K]`` (reference ``vq_qmm.py:93-152``)."""

    _check_impl(implementation)
    _validate_dims(in_dim, out_dim, group_size, code_bits)
    _check_dup(codebook_duplication)
    device = _device_of(x, codes, scales)
    xt = _to_dev(x, device)
    if xt.ndim != 2 or xt.shape[1] != in_dim:
        raise ValueError(f"x must have shape [M, {in_dim}], found {tuple(xt.shape)}")
    c = _codes_tensor(codes, code_bits, device)
    s = _to_dev(scales, device)
    if tuple(c.shape) != (out_dim, in_dim // 8):
        raise ValueError(f"codes must have shape ({out_dim}, {in_dim // 8}), found {tuple(c.shape)}")
    if tuple(s.shape) != (out_dim, in_dim // group_size):
        raise ValueError(f"scales must have shape ({out_dim}, {in_dim // group_size}), found {tuple(s.shape)}")
    cb = _codebook_tensor(codebook, code_bits, device)
    M = xt.shape[0]
    return routed_matvec(xt, c.reshape(1, out_dim, -1), s.reshape(1, out_dim, -1), cb, None, input_dims=in_dim,
                         output_dims=out_dim, group_size=group_size, code_bits=code_bits, routes=M)


# --------------------------------------------------------------------------- routed operators


def _validate_switch(x, codes, scales, codebook_t, *, input_dims, output_dims, group_size, code_bits):
    _validate_dims(input_dims, output_dims, group_size, code_bits)
    if x.shape[-1] != input_dims:
        raise ValueError(f"x trailing dimension must be {input_dims}, found {x.shape[-1]}")
    if codes.ndim != 3:
        raise ValueError(f"codes must be 3D [experts, out, in/8], found {tuple(codes.shape)}")
    if scales.ndim != 3:
        raise ValueError(f"scales must be 3D [experts, out, in/group], found {tuple(scales.shape)}")
    E = codes.shape[0]
    if tuple(codes.shape) != (E, output_dims, input_dims // 8):
        raise ValueError(f"codes must have shape {(E, output_dims, input_dims // 8)}, found {tuple(codes.shape)}")
    if tuple(scales.shape) != (E, output_dims, input_dims // group_size):
        raise ValueError(f"scales must have shape {(E, output_dims, input_dims // group_size)}, "
                         f"found {tuple(scales.shape)}")
    return E


def _host_check_indices(name: str, ix: torch.Tensor, upper: int) -> None:
    if ix.numel():
        lo, hi = int(ix.min()), int(ix.max())
        if lo < 0 or hi >= upper:
            raise ValueError(f"{name} must be in [0, {upper}), found range [{lo}, {hi}]")


def gather_vqmm(x, codes, scales, codebook, rhs_indices, *, lhs_indices=None, input_dims: int, output_dims: int,
                group_size: int = 512, code_bits: Literal[8, 16] = 8, codebook_duplication: Literal[1, 4, 8] = 1,
                implementation: str = "hip", sorted_indices: bool = False, route_strategy: str = "auto",
                validate_indices: bool = False) -> torch.Tensor:
    """Routed VQ gather-matmul (reference ``vq_switch.py:916-1221``).

    Token layout: ``x [T, K]``, ``rhs_indices [T, k]`` -> ``[T, k, N]``.
    Per-route layout: ``lhs_indices`` and ``rhs_indices`` of R routes -> ``[R, N]``.

    ``route_strategy="auto"``: E8P calls with 16-bit activations and at least
    ``GEMM_ROUTE_THRESHOLD`` routes (or ``sorted_indices``) take
    ``sorted_tiled`` -- the device route plan plus the MFMA grouped GEMM --
    everything else takes ``direct``, the wave-per-rows decode mat-vec.
    ``per_route_decoded`` is the same mat-vec (one launch for all routes).
    """

    _check_impl(implementation)
    _check_dup(codebook_duplication)
    if route_strategy not in ("auto", "direct", "sorted_tiled", "per_route_decoded"):
        raise ValueError("route_strategy must be 'auto', 'direct', 'sorted_tiled', or 'per_route_decoded'")
    device = _device_of(x, codes, scales, rhs_indices)
    xt = _to_dev(x, device)
    if xt.ndim != 2:
        raise ValueError(f"x must be 2D [tokens, hidden], found {tuple(xt.shape)}")
    rhs = _index_tensor(rhs_indices, device)
    if rhs.ndim not in (1, 2):
        raise ValueError(f"rhs_indices must be 1D or 2D, found {tuple(rhs.shape)}")
    c = _codes_tensor(codes, code_bits, device)
    s = _to_dev(scales, device)
    cb = _codebook_tensor(codebook, code_bits, device)
    E = _validate_switch(xt, c, s, cb, input_dims=input_dims, output_dims=output_dims, group_size=group_size,
                         code_bits=code_bits)
    if lhs_indices is not None:
        lhs = _index_tensor(lhs_indices, device).reshape(-1)
        flat_rhs = rhs.reshape(-1)
        if lhs.shape != flat_rhs.shape:
            raise ValueError("lhs_indices and rhs_indices must have the same flattened shape")
        out_shape = (flat_rhs.numel(), output_dims)
        x_div = 1
    else:
        if rhs.ndim != 2:
            raise ValueError("rhs_indices must be 2D [tokens, top_k] when lhs_indices is not provided")
        if rhs.shape[0] != xt.shape[0]:
            raise ValueError(f"rhs_indices token dimension {rhs.shape[0]} must match x token dimension "
                             f"{xt.shape[0]}")
        lhs = None
        flat_rhs = rhs.reshape(-1)
        x_div = rhs.shape[1]
        out_shape = (xt.shape[0], rhs.shape[1], output_dims)
    if validate_indices:
        _host_check_indices("rhs_indices", flat_rhs, E)
        if lhs is not None:
            _host_check_indices("lhs_indices", lhs, xt.shape[0])
    R = flat_rhs.numel()
    od = output_dtype(xt.dtype)
    if R == 0:
        return torch.zeros(out_shape, dtype=od, device=device)

    eligible = gemm_eligible(code_bits=code_bits, x_dtype=xt.dtype, input_dims=input_dims, group_size=group_size)
    strategy = route_strategy
    if strategy == "auto":
        strategy = "sorted_tiled" if eligible and (sorted_indices or R >= GEMM_ROUTE_THRESHOLD) else "direct"
    _trace(token_rows=int(xt.shape[0]), route_count=int(R), has_lhs_indices=lhs_indices is not None,
           input_dims=int(input_dims), output_dims=int(output_dims), group_size=int(group_size),
           code_bits=int(code_bits), strategy=strategy,
           implementation="mfma_grouped_gemm" if strategy == "sorted_tiled" and eligible else "hip_matvec")
    if strategy in ("direct", "per_route_decoded"):
        y = routed_matvec(xt, c, s, cb, flat_rhs, lhs=lhs, x_div=x_div, input_dims=input_dims,
                          output_dims=output_dims, group_size=group_size, code_bits=code_bits)
        return y.reshape(out_shape)
    # sorted_tiled
    full_lhs = lhs if lhs is not None else torch.arange(R, dtype=torch.int32, device=device) // x_div
    order, inverse, _, _, te, to, tc, _ = route_plan(flat_rhs, E, GEMM_ROUTE_TILE)
    sorted_lhs = full_lhs[order.long()].contiguous()
    if eligible:  # rows land in route order directly
        y = grouped_gemm(xt, c, s, cb, (te, to, tc), lhs=sorted_lhs, routes=R, input_dims=input_dims,
                         output_dims=output_dims, group_size=group_size, out_index=order)
        return y.reshape(out_shape)
    else:
        sorted_rhs = flat_rhs[order.long()].contiguous()
        routed = routed_matvec(xt, c, s, cb, sorted_rhs, lhs=sorted_lhs, input_dims=input_dims,
                               output_dims=output_dims, group_size=group_size, code_bits=code_bits)
    return routed[inverse.long()].reshape(out_shape)


def gather_vqmm_sorted_routes(x, codes, scales, codebook, sorted_rhs, sorted_lhs, *, input_dims: int,
                              output_dims: int, group_size: int = 512, code_bits: Literal[8, 16] = 8,
                              codebook_duplication: Literal[1, 4, 8] = 8, implementation: str = "hip",
                              projection: str = "auto", validate_indices: bool = False, tile_descriptors=None,
                              x_pre_sorted: bool = False) -> torch.Tensor:
    """Already-sorted routed matmul -> ``[R, N]`` in sorted order
    (reference ``vq_switch.py:620-913``). E8P with 16-bit activations runs the
    MFMA grouped GEMM (``tile_descriptors`` or a device route plan of 64-route
    tiles); other calls run the mat-vec over the sorted routes."""

    if projection not in ("auto", "gate_up", "down"):
        raise ValueError("projection must be 'auto', 'gate_up', or 'down'")
    if implementation not in ("hip", "metal", "auto", "nax_e8p", "nax_e8p_m32n64", "nax_e8"):
        _check_impl(implementation)
    _check_dup(codebook_duplication)
    device = _device_of(x, codes, scales, sorted_rhs)
    xt = _to_dev(x, device)
    rhs = _index_tensor(sorted_rhs, device).reshape(-1)
    lhs = _index_tensor(sorted_lhs, device).reshape(-1)
    if xt.ndim != 2:
        raise ValueError(f"x must be 2D [tokens_or_routes, input_dims], found {tuple(xt.shape)}")
    if xt.shape[1] != input_dims:
        raise ValueError(f"x trailing dimension must be {input_dims}, found {xt.shape[1]}")
    if rhs.shape != lhs.shape:
        raise ValueError("sorted_rhs and sorted_lhs must have the same flattened shape")
    c = _codes_tensor(codes, code_bits, device)
    s = _to_dev(scales, device)
    cb = _codebook_tensor(codebook, code_bits, device)
    E = _validate_switch(xt, c, s, cb, input_dims=input_dims, output_dims=output_dims, group_size=group_size,
                         code_bits=code_bits)
    R = rhs.numel()
    if R == 0:
        return torch.zeros((0, output_dims), dtype=output_dtype(xt.dtype), device=device)
    if validate_indices:
        _host_check_indices("sorted_rhs", rhs, E)
        _host_check_indices("sorted_lhs", lhs, xt.shape[0])
        if R > 1 and bool((rhs[1:] < rhs[:-1]).any()):
            raise ValueError("sorted_rhs must be sorted nondecreasing by expert id")
    if code_bits == 16 and xt.dtype == torch.float32:
        xt = xt.to(torch.float16)  # the reference's native path runs fp16 activations (vq_switch.py:758-761)
    skip_gather = x_pre_sorted and xt.shape[0] == R
    use_lhs = None if skip_gather else lhs
    if gemm_eligible(code_bits=code_bits, x_dtype=xt.dtype, input_dims=input_dims, group_size=group_size):
        if tile_descriptors is None:
            _, _, _, _, te, to, tc, _ = route_plan(rhs, E, GEMM_ROUTE_TILE)
        else:
            te, to, tc = (_index_tensor(t, device).reshape(-1) for t in tile_descriptors)
            if int(tc.max()) > GEMM_ROUTE_TILE:
                raise ValueError(f"tile_descriptors may hold at most {GEMM_ROUTE_TILE} routes per tile")
        return grouped_gemm(xt, c, s, cb, (te, to, tc), lhs=use_lhs, routes=R, input_dims=input_dims,
                            output_dims=output_dims, group_size=group_size)
    return routed_matvec(xt, c, s, cb, rhs, lhs=use_lhs if use_lhs is not None else None,
                         x_div=1, input_dims=input_dims, output_dims=output_dims, group_size=group_size,
                         code_bits=code_bits)


def verify_m_rows(route_count: int, top_k: int) -> int:
    """Row-tile width for expert-grouped verify (reference ``gather_vqmm.py:272-284``)."""

    verify_rows = max(1, route_count // max(1, top_k))
    for candidate in VERIFY_MROWS_VALUES:
        if candidate >= verify_rows:
            return candidate
    return 8


def gather_vqmm_verify_rows(x, codes, scales, codebook, rhs_indices, *, lhs_indices=None, input_dims: int,
                            output_dims: int, group_size: int = 512, grouping: str = "flat",
                            m_rows: int | str = "auto", rows_per_threadgroup: int | str = "auto") -> torch.Tensor:
    """Wide-M verify pass over routed experts (reference ``vq_switch.py:286-377``).

    The code format follows ``codes``' dtype: uint8 codes index a packed 8-bit
    E8 table (the reference kernel's contract, ``gather_vqmm.py:387-388``;
    default ``codebook`` the E8 table), uint16 codes are E8P.
    ``grouping="flat"``: one launch, every route on the decode mat-vec.
    ``grouping="expert"``: routes sorted by expert on the device and folded in
    tiles of up to ``m_rows`` same-expert routes that share every code load;
    per route bit-identical with ``"flat"``.
    """

    if grouping not in ("expert", "flat"):
        raise ValueError("grouping must be 'expert' or 'flat'")
    if rows_per_threadgroup != "auto" and (not isinstance(rows_per_threadgroup, int) or rows_per_threadgroup < 1):
        raise ValueError("rows_per_threadgroup must be 'auto' or a positive int")
    device = _device_of(x, codes, scales, rhs_indices)
    xt = _to_dev(x, device)
    if xt.ndim != 2:
        raise ValueError(f"x must be 2D [rows, input_dims], found {tuple(xt.shape)}")
    rhs = _index_tensor(rhs_indices, device)
    code_bits = _code_bits_of(codes)
    c = _codes_tensor(codes, code_bits, device)
    s = _to_dev(scales, device)
    cb = _codebook_tensor(codebook, code_bits, device)
    E = _validate_switch(xt, c, s, cb, input_dims=input_dims, output_dims=output_dims, group_size=group_size,
                         code_bits=code_bits)
    if lhs_indices is not None:
        flat_rhs = rhs.reshape(-1)
        flat_lhs = _index_tensor(lhs_indices, device).reshape(-1)
        if flat_lhs.shape != flat_rhs.shape:
            raise ValueError("lhs_indices and rhs_indices must have the same flattened shape")
        out_shape = (flat_rhs.numel(), output_dims)
        top_k = None
    else:
        if rhs.ndim != 2:
            raise ValueError("rhs_indices must be 2D [verify_rows, top_k] when lhs_indices is not provided")
        if rhs.shape[0] != xt.shape[0]:
            raise ValueError(f"rhs_indices row dimension {rhs.shape[0]} must match x row dimension {xt.shape[0]}")
        top_k = rhs.shape[1]
        flat_rhs = rhs.reshape(-1)
        flat_lhs = torch.arange(flat_rhs.numel(), dtype=torch.int32, device=device) // top_k
        out_shape = (xt.shape[0], top_k, output_dims)
    R = flat_rhs.numel()
    if R == 0:
        return torch.zeros(out_shape, dtype=output_dtype(xt.dtype), device=device)
    if m_rows == "auto":
        mr = verify_m_rows(R, top_k) if top_k is not None else _VERIFY_DEFAULT_M_ROWS
    else:
        if m_rows not in VERIFY_MROWS_VALUES:
            raise ValueError(f"m_rows must be one of {VERIFY_MROWS_VALUES}")
        mr = int(m_rows)
    _trace(token_rows=int(xt.shape[0]), route_count=int(R), has_lhs_indices=lhs_indices is not None,
           input_dims=int(input_dims), output_dims=int(output_dims), group_size=int(group_size),
           code_bits=code_bits, strategy=f"verify_{grouping}", implementation="hip_matvec")
    if grouping == "flat":
        y = routed_matvec(xt, c, s, cb, flat_rhs, lhs=flat_lhs, input_dims=input_dims, output_dims=output_dims,
                          group_size=group_size, code_bits=code_bits)
        return y.reshape(out_shape)
    order, inverse, _, _, te, to, tc, _ = route_plan(flat_rhs, E, mr)
    sorted_lhs = flat_lhs[order.long()].contiguous()
    routed = torch.empty((R, output_dims), dtype=output_dtype(xt.dtype), device=device)
    _lib.call("keep_vq_matvec_tiles", xt.data_ptr(), _dtype_code(xt, "x"), xt.shape[0], c.data_ptr(), code_bits,
              s.data_ptr(), _dtype_code(s, "scales"), cb.data_ptr(), sorted_lhs.data_ptr(), R, te.data_ptr(),
              to.data_ptr(), tc.data_ptr(), te.numel(), mr, E, output_dims, input_dims, group_size,
              routed.data_ptr(), _DT[routed.dtype], _stream(device))
    return routed[inverse.long()].reshape(out_shape)


# --------------------------------------------------------------------------- e8p_m1 / nested


def _m1_args(rows_per_simdgroup: int, simdgroups: int) -> None:
    if rows_per_simdgroup < 1 or simdgroups < 1 or simdgroups > 32:
        raise ValueError("rows_per_simdgroup must be >= 1 and simdgroups in 1..32")


def _e8p_inputs(x, codes, scales, codebook, rhs_indices, output_dims):
    device = _device_of(x, codes, scales, rhs_indices)
    xt = _to_dev(x, device)
    c = _codes_tensor(codes, 16, device)
    s = _to_dev(scales, device)
    cb = _codebook_tensor(codebook, 16, device)
    rhs = _index_tensor(rhs_indices, device)
    if c.ndim != 3 or c.shape[1] != output_dims:
        raise ValueError(f"codes must be [experts, {output_dims}, in/8], found {tuple(c.shape)}")
    K = c.shape[2] * 8
    if xt.ndim != 2 or xt.shape[1] != K:
        raise ValueError(f"x must be [rows, {K}], found {tuple(xt.shape)}")
    if s.ndim != 3 or s.shape[:2] != c.shape[:2] or c.shape[2] % s.shape[2]:
        raise ValueError(f"scales must be [experts, {output_dims}, groups] dividing {c.shape[2]} codewords")
    gs = K // s.shape[2]
    if gs % 8:
        raise ValueError("codewords per scale group must be whole codewords")
    return xt, c, s, cb, rhs, K, gs


def e8p_m1_token_layout(x, codes, scales, codebook, rhs_indices, *, output_dims: int, rows_per_simdgroup: int = 4,
                        simdgroups: int = 1) -> torch.Tensor:
    """Token ``t``'s row against its ``top_k`` experts -> ``[T, k, N]``
    (reference ``e8p_m1.py:134-157``)."""

    _m1_args(rows_per_simdgroup, simdgroups)
    xt, c, s, cb, rhs, K, gs = _e8p_inputs(x, codes, scales, codebook, rhs_indices, output_dims)
    if rhs.ndim != 2 or rhs.shape[0] != xt.shape[0]:
        raise ValueError("token-layout E8P needs x [tokens, in] and rhs_indices [tokens, top_k]")
    T, k = rhs.shape
    y = routed_matvec(xt, c, s, cb, rhs.reshape(-1), x_div=k, input_dims=K, output_dims=output_dims, group_size=gs)
    return y.reshape(T, k, output_dims)


def e8p_m1_per_route(x, codes, scales, codebook, rhs_indices, *, output_dims: int, rows_per_simdgroup: int = 4,
                     simdgroups: int = 1) -> torch.Tensor:
    """Route ``r``'s row against expert ``rhs_indices[r]`` -> ``[R, N]``
    (reference ``e8p_m1.py:160-183``)."""

    _m1_args(rows_per_simdgroup, simdgroups)
    xt, c, s, cb, rhs, K, gs = _e8p_inputs(x, codes, scales, codebook, rhs_indices, output_dims)
    R = rhs.numel()
    if xt.ndim != 2 or xt.shape[0] != R:
        raise ValueError(f"per-route E8P M=1 needs x [{R}, in], got {tuple(xt.shape)}")
    return routed_matvec(xt, c, s, cb, rhs.reshape(-1), x_div=1, input_dims=K, output_dims=output_dims,
                         group_size=gs)


def _nested_inputs(x, base, rhs_indices, residual, hot_of_slot, output_dims):
    codes, scales, codebook = base
    res_codes, res_scales, res_table = residual
    xt, c, s, cb, rhs, K, gs = _e8p_inputs(x, codes, scales, codebook, rhs_indices, output_dims)
    device = xt.device
    rc = _codes_tensor(res_codes, 8, device)
    if tuple(rc.shape[1:]) != tuple(c.shape[1:]):
        raise ValueError(f"base and residual rows differ: {tuple(c.shape[1:])} and {tuple(rc.shape[1:])}")
    rs = _to_dev(res_scales, device)
    rt = _to_dev(res_table, device)
    if tuple(rt.shape) != (256, 4):
        raise ValueError("the residual table must be half2_pairs(grid): [256, 4] uint32")
    hot = _to_dev(hot_of_slot, device)
    if hot.numel() != c.shape[0]:
        raise ValueError(f"hot_of_slot needs one entry per slot, got {hot.numel()} for {c.shape[0]}")
    if hot.dtype not in (torch.int32, torch.int64):
        raise ValueError("hot_of_slot must be uint32")
    hot = hot.to(torch.int64).bitwise_and(0xFFFFFFFF).to(torch.int64)
    hot32 = torch.where(hot == NO_RESIDUAL, torch.full_like(hot, -1), hot).to(torch.int32).contiguous()
    return xt, c, s, cb, rhs, K, gs, (rc, rs, rt), hot32


def e8p_nested_m1_token_layout(x, base, rhs_indices, residual, hot_of_slot, *, output_dims: int,
                               rows_per_simdgroup: int = 4, simdgroups: int = 1) -> torch.Tensor:
    """Nested tier, token layout (reference ``e8p_nested_m1.py:90-100``):
    ``base`` / ``residual`` are ``(codes, scales, table)``; ``hot_of_slot[slot]``
    is the residual row or ``0xFFFFFFFF``."""

    _m1_args(rows_per_simdgroup, simdgroups)
    xt, c, s, cb, rhs, K, gs, res, hot = _nested_inputs(x, base, rhs_indices, residual, hot_of_slot, output_dims)
    if rhs.ndim != 2 or rhs.shape[0] != xt.shape[0]:
        raise ValueError("token-layout nested E8P needs x [tokens, in] and rhs_indices [tokens, top_k]")
    T, k = rhs.shape
    y = routed_matvec(xt, c, s, cb, rhs.reshape(-1), x_div=k, input_dims=K, output_dims=output_dims, group_size=gs,
                      residual=res, hot_of_slot=hot)
    return y.reshape(T, k, output_dims)


def e8p_nested_m1_per_route(x, base, rhs_indices, residual, hot_of_slot, *, output_dims: int,
                            rows_per_simdgroup: int = 4, simdgroups: int = 1) -> torch.Tensor:
    """Nested tier, per-route layout (reference ``e8p_nested_m1.py:103-112``)."""

    _m1_args(rows_per_simdgroup, simdgroups)
    xt, c, s, cb, rhs, K, gs, res, hot = _nested_inputs(x, base, rhs_indices, residual, hot_of_slot, output_dims)
    R = rhs.numel()
    if xt.shape[0] != R:
        raise ValueError(f"per-route nested E8P needs x [{R}, in], got {tuple(xt.shape)}")
    return routed_matvec(xt, c, s, cb, rhs.reshape(-1), x_div=1, input_dims=K, output_dims=output_dims,
                         group_size=gs, residual=res, hot_of_slot=hot)


# --------------------------------------------------------------------------- e8_1bit_m1 (residual tier alone)


def pair_packed(packed) -> np.ndarray:
    """The packed 8-bit E8 table (nibble d = dim d) with dims 2k and 2k + 1 in
    nibbles k and k + 4 (reference ``e8_1bit_m1.py:25-33``)."""

    p = np.asarray(packed, dtype=np.uint32)
    out = np.zeros(p.shape, np.uint32)
    for k in range(4):
        out |= ((p >> np.uint32(8 * k)) & np.uint32(0xF)) << np.uint32(4 * k)
        out |= ((p >> np.uint32(8 * k + 4)) & np.uint32(0xF)) << np.uint32(16 + 4 * k)
    return out


_UNPAIRED: dict = {}


def _unpaired_table(codebook: torch.Tensor) -> torch.Tensor:
    """The inverse of ``pair_packed`` on a device table (nibble d = dim d), cached
    per table tensor."""

    key = (codebook.data_ptr(), str(codebook.device))
    hit = _UNPAIRED.get(key)
    if hit is not None and hit[0] is codebook:
        return hit[1]
    p = codebook.to(torch.int64) & 0xFFFFFFFF
    out = torch.zeros_like(p)
    for k in range(4):
        out |= ((p >> (4 * k)) & 0xF) << (8 * k)
        out |= ((p >> (16 + 4 * k)) & 0xF) << (8 * k + 4)
    t = (out - ((out >> 31) << 32)).to(torch.int32).contiguous()  # the same bits as int32
    _UNPAIRED[key] = (codebook, t)
    return t


def _route_bits(rhs_indices, device) -> torch.Tensor:
    """Route indices as int32 holding the uint32 bits (``NO_RESIDUAL`` -> -1), flat."""

    if isinstance(rhs_indices, torch.Tensor) and rhs_indices.dtype == torch.int32:
        return rhs_indices.to(device).reshape(-1).contiguous()
    if isinstance(rhs_indices, torch.Tensor) and rhs_indices.dtype == torch.int64:
        r = rhs_indices.to(device) & 0xFFFFFFFF
        return (r - ((r >> 31) << 32)).to(torch.int32).reshape(-1).contiguous()
    a = rhs_indices.cpu().numpy() if isinstance(rhs_indices, torch.Tensor) else np.asarray(rhs_indices)
    a = a.astype(np.int64) & 0xFFFFFFFF
    return torch.from_numpy(a.astype(np.uint32).view(np.int32).reshape(-1).copy()).to(device)


def _e8_1bit_launch(x, codes, scales, codebook, rhs_indices, output_dims: int, x_div: int,
                    rows_per_simdgroup: int, simdgroups: int) -> torch.Tensor:
    _m1_args(rows_per_simdgroup, simdgroups)
    device = _device_of(x, codes, scales, rhs_indices)
    xt = _to_dev(x, device).contiguous()
    c = _codes_tensor(codes, 8, device)
    s = _to_dev(scales, device)
    if c.ndim != 3 or c.shape[1] != output_dims:
        raise ValueError(f"codes must be [experts, {output_dims}, in/8], found {tuple(c.shape)}")
    K = c.shape[2] * 8
    if xt.ndim != 2 or xt.shape[1] != K:
        raise ValueError(f"x must be [rows, {K}], found {tuple(xt.shape)}")
    if s.ndim != 3 or s.shape[:2] != c.shape[:2] or c.shape[2] % s.shape[2]:
        raise ValueError(f"scales must be [experts, {output_dims}, groups] dividing {c.shape[2]} codewords")
    if codebook is None:
        cb = _to_dev(e8_1bit_packed().view(np.int32), device)
    else:
        t = _to_dev(codebook, device)
        if t.numel() != 256 or str(t.dtype).rsplit(".", 1)[-1] not in ("uint32", "int32"):
            raise ValueError("the 8-bit E8 table must be 256 uint32 entries in pair_packed layout")
        cb = _unpaired_table(t.reshape(256))
    rhs = _route_bits(rhs_indices, device)
    R = rhs.numel()
    out = torch.empty((R, output_dims), dtype=output_dtype(xt.dtype), device=device)
    if R == 0:
        return out
    _lib.call("keep_e8_1bit_matvec", xt.data_ptr(), _dtype_code(xt, "x"), xt.shape[0], c.data_ptr(), s.data_ptr(),
              _dtype_code(s, "scales"), cb.data_ptr(), rhs.data_ptr(), R, x_div, c.shape[0], output_dims, K,
              K // s.shape[2], out.data_ptr(), _DT[out.dtype], _stream(device))
    return out


def e8_1bit_m1_token_layout(x, codes, scales, codebook, rhs_indices, *, output_dims: int,
                            rows_per_simdgroup: int = 4, simdgroups: int = 1) -> torch.Tensor:
    """8-bit E8 residual alone, token layout -> ``[T, k, N]``; a route index of
    ``NO_RESIDUAL`` writes zeros (reference ``e8_1bit_m1.py:76-85``).
    ``codebook`` is the ``pair_packed`` table (``None``: the default one)."""

    shape = tuple(rhs_indices.shape)
    if x.ndim != 2 or len(shape) != 2 or shape[0] != x.shape[0]:
        raise ValueError("token-layout E8 needs x [tokens, in] and rhs_indices [tokens, top_k]")
    T, k = shape
    rhs = rhs_indices
    y = _e8_1bit_launch(x, codes, scales, codebook, rhs, output_dims, k, rows_per_simdgroup, simdgroups)
    return y.reshape(T, k, output_dims)


def e8_1bit_m1_per_route(x, codes, scales, codebook, rhs_indices, *, output_dims: int,
                         rows_per_simdgroup: int = 4, simdgroups: int = 1) -> torch.Tensor:
    """8-bit E8 residual alone, per-route layout -> ``[R, N]``; ``NO_RESIDUAL``
    routes write zeros (reference ``e8_1bit_m1.py:88-97``)."""

    R = int(np.prod(tuple(rhs_indices.shape)))
    if x.ndim != 2 or x.shape[0] != R:
        raise ValueError(f"per-route E8 needs x [{R}, in], got {tuple(x.shape)}")
    return _e8_1bit_launch(x, codes, scales, codebook, rhs_indices, output_dims, 1, rows_per_simdgroup,
                           simdgroups)
