"""The steps either side of the routed experts on the GPU.

- ``rmsnorm_quant_rht``: RMSNorm, block-wise FP8 e4m3 activation quantisation
  and the forward RHT in one row pass (``keep_rmsnorm_quant_rht``): the
  block's ``ffn_norm`` (``src/ramp/models/deepseek_v4_flash_adapter.py:1794,1806``),
  ``act_quant`` (``scripts/runpod/v41_reap/torch_kernel.py:40-53``), whose
  values the serving step feeds to the experts
  (``scripts/v41_build/omlx_lattice.py:332,357``), and ``apply_rht_mx``
  (``src/keep/quant/rht.py:84-91``).
- ``combine_add``: the routed sum plus the shared expert plus the residual,
  rounded once (``keep_moe_combine_add``; ``deepseek_v4_flash_adapter.py:1784``,
  ``omlx_lattice.py:374-388``).
"""

from __future__ import annotations

import torch

from keep_amd import _lib


def rmsnorm_quant_rht(x: torch.Tensor, gamma: torch.Tensor | None = None, eps: float = 1e-6, *,
                      quant_block: int = 128, pow2_scales: bool = False, rht_signs=None, return_normed: bool = False,
                      out_dtype: torch.dtype | None = None, validate_signs: bool = True):
    """``y = RMSNorm(x)`` (rounded to ``x``'s dtype), ``q = act_quant(y)`` per
    ``quant_block`` values (0: none), ``out = RHT(q, rht_signs)`` (no signs: q).
    Returns ``out`` or ``(out, y)`` with ``return_normed``."""

    from keep_amd.ops import _DT, _stream
    from keep_amd.rht import check_signs

    if not x.is_cuda:
        raise ValueError("rmsnorm_quant_rht needs a device tensor")
    if x.dtype not in _DT:
        raise ValueError(f"x must be float32, float16 or bfloat16, found {x.dtype}")
    n = x.shape[-1]
    if n < 64 or n > 8192 or n & (n - 1):
        raise ValueError(f"rows must hold a power of two of 64..8192 values, found {n}")
    if quant_block and (quant_block < 16 or quant_block > min(1024, n) or quant_block & (quant_block - 1)):
        raise ValueError(f"quant_block must be 0 or a power of two in 16..{min(1024, n)}, found {quant_block}")
    od = out_dtype or x.dtype
    if od not in _DT:
        raise ValueError(f"unsupported output dtype {od}")
    g = None
    if gamma is not None:
        g = gamma.to(device=x.device).contiguous()
        if g.dtype not in _DT:
            g = g.float()
        if tuple(g.shape) != (n,):
            raise ValueError(f"gamma must have shape ({n},), found {tuple(g.shape)}")
    s = None
    if rht_signs is not None:
        s = torch.as_tensor(rht_signs, device=x.device).to(torch.float32).contiguous()
        if tuple(s.shape) != (n,):
            raise ValueError(f"rht_signs must have shape ({n},), found {tuple(s.shape)}")
        if validate_signs:
            check_signs(s)
    xc = x.contiguous()
    rows = xc.numel() // n
    out = torch.empty(x.shape, dtype=od, device=x.device)
    normed = torch.empty(x.shape, dtype=x.dtype, device=x.device) if return_normed else None
    _lib.call("keep_rmsnorm_quant_rht", xc.data_ptr(), _DT[xc.dtype], rows, n, None if g is None else g.data_ptr(),
              _DT[g.dtype] if g is not None else 0, float(eps), int(quant_block), int(bool(pow2_scales)),
              None if s is None else s.data_ptr(), None if normed is None else normed.data_ptr(), out.data_ptr(),
              _DT[od], _stream(x.device))
    return (out, normed) if return_normed else out


def combine_add(routed: torch.Tensor, shared: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``round_out(residual + (routed + shared))`` with fp32 sums; ``routed`` is float32."""

    from keep_amd.ops import _DT, _stream

    if routed.dtype != torch.float32 or not routed.is_cuda:
        raise ValueError("routed must be a float32 device tensor")
    for name, t in (("shared", shared), ("residual", residual)):
        if t is not None and (tuple(t.shape) != tuple(routed.shape) or t.dtype not in _DT):
            raise ValueError(f"{name} must match routed's shape {tuple(routed.shape)} in a float dtype")
    od = out_dtype or (residual.dtype if residual is not None else torch.float32)
    r = routed.contiguous()
    sh = None if shared is None else shared.contiguous()
    rs = None if residual is None else residual.contiguous()
    out = torch.empty(routed.shape, dtype=od, device=routed.device)
    _lib.call("keep_moe_combine_add", r.data_ptr(), None if sh is None else sh.data_ptr(),
              _DT[sh.dtype] if sh is not None else 0, None if rs is None else rs.data_ptr(),
              _DT[rs.dtype] if rs is not None else 0, r.numel(), out.data_ptr(), _DT[od], _stream(routed.device))
    return out
