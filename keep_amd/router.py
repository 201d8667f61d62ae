"""Residency-biased dual top-k router on the GPU (``keep_router_dual_topk``).

One evaluation per token gives both the *served* top-k (over
``score + bias_served``; absent experts carry a bias <= -1e30, the serving
cache's ``OFF``) and the *demand* top-k (over ``score + bias_demand``, the
unmasked pool), as the reference's dual top-k kernel
(``scripts/v41_build/omlx_lattice.py:77-97``) and ``gate_masked``
(``scripts/runpod/v41_reap/local_eval.py:69-91``) define them. Ties are broken
by the lower expert index; the order of the k slots is descending key.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from keep_amd import _lib
from keep_amd.ops import _device_of, _ptr, _stream, _to_dev

OFF = -1.0e30  # bias of an absent expert (reference omlx_routed.py:40)


class RouterOutput(NamedTuple):
    idx: torch.Tensor  # [T, k] int32 served experts
    weight: torch.Tensor  # [T, k] float32 routing weights (0 for an absent pick)
    want: torch.Tensor  # [T, k] int32 demanded experts
    want_score: torch.Tensor  # [T, k] float32 raw scores of the demand
    admit: torch.Tensor  # [T, k] uint8: demanded, absent and normalised weight >= tau


def router_dual_topk(logits, k: int, *, bias_served=None, bias_demand=None, score_func: str = "softmax",
                     renormalize: bool = True, route_scale: float = 1.0, tau: float = float("inf"),
                     slot_map=None, num_slots: int | None = None) -> RouterOutput:
    """Served and demanded top-k from one router evaluation.

    ``logits [T, E]`` are cast to float32. ``bias_served`` holds the score
    correction bias plus the residency mask (``OFF`` for absent experts);
    ``bias_demand`` the correction bias alone. Weights are the served scores
    (0 for an absent pick), renormalised to sum 1 (``+1e-20``) when
    ``renormalize``, times ``route_scale``. With ``slot_map`` (int32 ``[E]``,
    expert -> row of a pool of ``num_slots`` rows) ``idx`` holds the served
    experts' rows (-1 outside the pool), as the serving router's
    ``slot_of[chosen]`` (``omlx_lattice.py:77-97``); ``want`` stays expert ids.
    """

    if score_func not in _lib.SCORE_FUNCS:
        raise ValueError(f"score_func must be one of {sorted(_lib.SCORE_FUNCS)}")
    device = _device_of(logits, bias_served, bias_demand)
    z = _to_dev(logits, device, torch.float32)
    if z.ndim != 2:
        raise ValueError(f"logits must be 2D [tokens, experts], found {tuple(z.shape)}")
    T, E = z.shape
    if not 1 <= k <= min(32, E):
        raise ValueError(f"k must be in 1..min(32, {E})")
    bs = None if bias_served is None else _to_dev(bias_served, device, torch.float32).reshape(-1)
    bd = None if bias_demand is None else _to_dev(bias_demand, device, torch.float32).reshape(-1)
    for name, b in (("bias_served", bs), ("bias_demand", bd)):
        if b is not None and b.numel() != E:
            raise ValueError(f"{name} must have {E} entries, found {b.numel()}")
    sm, ns = _slot_args(slot_map, num_slots, E, device)
    i32 = dict(dtype=torch.int32, device=device)
    f32 = dict(dtype=torch.float32, device=device)
    out = RouterOutput(torch.empty((T, k), **i32), torch.empty((T, k), **f32), torch.empty((T, k), **i32),
                       torch.empty((T, k), **f32), torch.empty((T, k), dtype=torch.uint8, device=device))
    if T == 0:
        return out
    _lib.call("keep_router_dual_topk", z.data_ptr(), T, E, k, _ptr(bs), _ptr(bd), _lib.SCORE_FUNCS[score_func],
              int(bool(renormalize)), float(route_scale), float(tau), _ptr(sm), ns, out.idx.data_ptr(),
              out.weight.data_ptr(), out.want.data_ptr(), out.want_score.data_ptr(), out.admit.data_ptr(),
              _stream(device))
    return out


def _slot_args(slot_map, num_slots, E: int, device):
    """``(slot_map int32 [E] on device or None, num_slots)`` for the C ABI."""

    if slot_map is None:
        return None, 0
    sm = _to_dev(slot_map, device, torch.int32).reshape(-1).contiguous()
    if sm.numel() != E:
        raise ValueError(f"slot_map must have {E} entries, found {sm.numel()}")
    if num_slots is None or num_slots < 1:
        raise ValueError("a slot_map needs num_slots >= 1 (the pool's rows)")
    return sm, int(num_slots)


def expert_select(logits, e_score_correction_bias, top_k: int, routed_scaling_factor: float, norm_topk_prob: bool,
                  scoring_func: str):
    """Drop-in for ``_expert_select`` (``deepseek_v4_flash_adapter.py:923-940``):
    top-k on ``score + bias``, weights = unbiased scores of the chosen experts,
    renormalised only for non-softmax scoring with ``norm_topk_prob``, times
    ``routed_scaling_factor``. Returns ``(inds int32 [T, k], weights float32 [T, k])``."""

    r = router_dual_topk(logits, top_k, bias_served=e_score_correction_bias, bias_demand=None,
                         score_func=scoring_func, renormalize=(scoring_func != "softmax" and norm_topk_prob),
                         route_scale=routed_scaling_factor)
    return r.idx, r.weight


def resident_bias(resident_mask, correction_bias=None) -> torch.Tensor:
    """``bias_served`` for a residency mask: ``OFF`` on absent experts, the
    correction bias (or 0) elsewhere."""

    m = resident_mask if isinstance(resident_mask, torch.Tensor) else torch.as_tensor(resident_mask)
    m = m.to(torch.bool)
    base = torch.zeros(m.shape, dtype=torch.float32, device=m.device) if correction_bias is None else \
        correction_bias.to(torch.float32).to(m.device)
    return torch.where(m, base, torch.full_like(base, OFF))
