"""Dense float64 reference of every routed-E8P hot-path operator -- CPU oracle
(test infrastructure only; see ``oracle/__init__.py``).

Every projection here materialises the dense weight matrix exactly as the
reference's oracle does (``src/ramp/kernels/vq_qmv.py:126-160``,
``vq_qmm.py:69-90``) but accumulates in float64, so the comparison with an
fp32-accumulating kernel is not blurred by an unspecified BLAS summation order.

Pins (``tests/test_oracle_ops.py``): brute-force scalar loops at tiny shapes,
linearity, permutation invariants of the route plan, and the router semantics
of the reference's ``tests/test_runpod_v41_routed_precision.py:158-179``.
"""

from __future__ import annotations

import numpy as np

from oracle.e8p import decode_weight_matrix

NO_RESIDUAL = 0xFFFFFFFF
MASKED_BIAS = -1.0e30  # an expert whose served-bias is <= this is absent (``omlx_routed.py:40``)


# --------------------------------------------------------------------------- projections


def dense(codes, scales, *, code_bits=16, table=None) -> np.ndarray:
    """Dequantised float64 weights ``[..., N, K]`` (value x scale is exact)."""

    return decode_weight_matrix(np.asarray(codes), np.asarray(scales, dtype=np.float64),
                                code_bits=code_bits, table=table, dtype=np.float64)


def qmv(x, codes, scales, *, code_bits=16, table=None) -> np.ndarray:
    """``y = W x`` for one matrix (``vq_qmv.py:126-160``); float64."""

    return dense(codes, scales, code_bits=code_bits, table=table) @ np.asarray(x, dtype=np.float64)


def qmm(x, codes, scales, *, code_bits=16, table=None) -> np.ndarray:
    """``Y = X W^T`` (``vq_qmm.py:69-90``); float64."""

    return np.asarray(x, dtype=np.float64) @ dense(codes, scales, code_bits=code_bits, table=table).T


class _ExpertCache:
    """Decode each touched expert once."""

    def __init__(self, codes, scales, code_bits, table):
        self.codes, self.scales, self.code_bits, self.table = codes, scales, code_bits, table
        self.w: dict[int, np.ndarray] = {}

    def __getitem__(self, e: int) -> np.ndarray:
        e = int(e)
        if e not in self.w:
            self.w[e] = dense(self.codes[e], self.scales[e], code_bits=self.code_bits, table=self.table)
        return self.w[e]


def gather_token(x, codes, scales, rhs, *, code_bits=16, table=None) -> np.ndarray:
    """Token layout ``x[T,K]``, ``rhs[T,k]`` -> ``[T,k,N]`` (``vq_switch.py:547-617``)."""

    x = np.asarray(x, dtype=np.float64)
    rhs = np.asarray(rhs)
    W = _ExpertCache(codes, scales, code_bits, table)
    T, k = rhs.shape
    N = np.asarray(codes).shape[1]
    out = np.zeros((T, k, N))
    for t in range(T):
        for j in range(k):
            out[t, j] = W[rhs[t, j]] @ x[t]
    return out


def gather_routes(x, codes, scales, rhs, lhs, *, code_bits=16, table=None) -> np.ndarray:
    """Per-route layout: route r multiplies ``x[lhs[r]]`` by expert ``rhs[r]`` -> ``[R,N]``."""

    x = np.asarray(x, dtype=np.float64)
    rhs = np.asarray(rhs).reshape(-1)
    lhs = np.asarray(lhs).reshape(-1)
    W = _ExpertCache(codes, scales, code_bits, table)
    N = np.asarray(codes).shape[1]
    out = np.zeros((rhs.shape[0], N))
    for r in range(rhs.shape[0]):
        out[r] = W[rhs[r]] @ x[lhs[r]]
    return out


def nested_routes(x, base, residual, hot_of_slot, rhs, lhs) -> np.ndarray:
    """Base E8P plus optional 8-bit E8 residual per slot
    (``src/ramp/kernels/e8p_nested_m1.metal:1-128``): ``hot_of_slot[slot]`` is the
    slot's row in the residual arrays or ``NO_RESIDUAL``."""

    (codes, scales), (rcodes, rscales) = base, residual
    y = gather_routes(x, codes, scales, rhs, lhs, code_bits=16)
    hot = np.asarray(hot_of_slot).astype(np.uint64)
    x = np.asarray(x, dtype=np.float64)
    R = _ExpertCache(rcodes, rscales, 8, None)
    for r, (s, t) in enumerate(zip(np.asarray(rhs).reshape(-1), np.asarray(lhs).reshape(-1))):
        h = int(hot[int(s)])
        if h != NO_RESIDUAL:
            y[r] += R[h] @ x[t]
    return y


# --------------------------------------------------------------------------- router


def score(logits, func: str = "softmax") -> np.ndarray:
    """Score function (``deepseek_v4_flash_adapter.py:913-921``), float64."""

    z = np.asarray(logits, dtype=np.float64)
    if func == "softmax":
        m = z.max(axis=-1, keepdims=True)
        e = np.exp(z - m)
        return e / e.sum(axis=-1, keepdims=True)
    if func == "sigmoid":
        return 1.0 / (1.0 + np.exp(-z))
    if func == "sqrtsoftplus":
        return np.sqrt(np.logaddexp(0.0, z))
    raise ValueError(f"unknown score function {func!r}")


def topk_rule(keys: np.ndarray, k: int) -> np.ndarray:
    """Top-k per row: larger key first, ties to the lower index. NaN ranks lowest."""

    keys = np.asarray(keys, dtype=np.float64)
    safe = np.where(np.isnan(keys), -np.inf, keys)
    E = safe.shape[-1]
    # lexsort: last key is primary -> sort by (-key, index)
    out = np.empty(safe.shape[:-1] + (k,), dtype=np.int64)
    for t in np.ndindex(safe.shape[:-1]):
        order = np.lexsort((np.arange(E), -safe[t]))
        out[t] = order[:k]
    return out


def router_dual_topk(logits, bias_served, bias_demand, k, *, func="softmax", renormalize=True,
                     route_scale=1.0, tau=float("inf")):
    """One router evaluation -> served and demanded top-k.

    Follows ``gate_masked`` (``scripts/runpod/v41_reap/local_eval.py:69-91``) and the
    dual top-k kernel (``scripts/v41_build/omlx_lattice.py:77-97``):

    - served = top-k of ``score + bias_served``; an expert with
      ``bias_served <= -1e30`` is absent and gets weight 0 if picked;
    - weights = scores of the served set (0 for absent), renormalised to sum 1
      (``+1e-20``) when ``renormalize``, times ``route_scale``;
    - demand = top-k of ``score + bias_demand`` with the raw scores;
    - admit = demanded expert absent and its normalised demand weight
      ``>= tau`` (``omlx_routed.py:186-193``).
    """

    s = score(logits, func)
    bs = np.asarray(bias_served, dtype=np.float64)
    bd = np.asarray(bias_demand, dtype=np.float64)
    absent = bs <= MASKED_BIAS
    idx = topk_rule(s + bs, k)
    w = np.take_along_axis(s, idx, axis=-1) * (~absent[idx])
    if renormalize:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    w = w * route_scale
    want = topk_rule(s + bd, k)
    want_score = np.take_along_axis(s, want, axis=-1)
    share = want_score / (want_score.sum(axis=-1, keepdims=True) + 1e-20) * route_scale
    admit = absent[want] & (share >= tau)
    return idx, w, want, want_score, admit


# --------------------------------------------------------------------------- SwiGLU / MoE


def swiglu(gate, up, limit: float = 0.0) -> np.ndarray:
    """``silu(min(g, L)) * clip(u, -L, L)``; plain SwiGLU when ``L <= 0``
    (``deepseek_v4_flash_adapter.py:962-967``)."""

    g = np.asarray(gate, dtype=np.float64)
    u = np.asarray(up, dtype=np.float64)
    if limit and limit > 0:
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
    return g / (1.0 + np.exp(-g)) * u


BF16_MAX = (2.0 - 2.0 ** -7) * 2.0 ** 127


def round_bf16(a) -> np.ndarray:
    """Round float32 or float64 values once to bfloat16 (nearest, ties to even;
    beyond the largest finite value to +-inf; subnormals on the 2^-133 grid),
    returned as float64. The step is 2^(e - 7) for |a| in [2^e, 2^(e+1)), and
    ``np.round`` of the exact quotient by it rounds half to even."""

    with np.errstate(invalid="ignore"):  # NaN payloads widen quietly
        x = np.asarray(a, dtype=np.float64)
    _, ex = np.frexp(x)  # |x| in [2^(ex-1), 2^ex)
    step = np.ldexp(1.0, np.maximum(ex - 8, -133))
    with np.errstate(invalid="ignore", over="ignore"):
        r = np.round(x / step) * step
        r = np.where(np.abs(r) > BF16_MAX, np.copysign(np.inf, x), r)
    return np.where(np.isfinite(x), r, x)


def moe_layer(x, idx, w, gate, up, down, *, limit=0.0, h_round=None, hot_of_slot=None,
              residual=None) -> np.ndarray:
    """Routed MoE: ``out[t] = sum_j w[t,j] * down_e(swiglu(gate_e x_t, up_e x_t))``
    with ``e = idx[t,j]`` (``glm4_moe_adapter.py:367-372``,
    ``deepseek_v4_flash_adapter.py:1776-1784``).

    ``gate``/``up``/``down`` are ``(codes, scales)`` pairs. ``h_round`` (a numpy
    dtype such as float16, or ``"bfloat16"``) rounds the SwiGLU output as a
    kernel that stores it in that dtype would (the reference's decode step
    stores it as bf16, ``scripts/v41_build/omlx_lattice.py:368``). ``residual`` is an optional dict ``{"gate": (rc, rs), ...}``
    of 8-bit residual tiers indexed through ``hot_of_slot``.
    """

    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(idx)
    w = np.asarray(w, dtype=np.float64)
    T, k = idx.shape
    Wg = _ExpertCache(*gate, 16, None)
    Wu = _ExpertCache(*up, 16, None)
    Wd = _ExpertCache(*down, 16, None)
    res = {}
    if residual is not None:
        res = {name: _ExpertCache(*residual[name], 8, None) for name in residual}
    hot = None if hot_of_slot is None else np.asarray(hot_of_slot).astype(np.uint64)
    H = np.asarray(down[0]).shape[1]
    out = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            e = int(idx[t, j])
            hrow = int(hot[e]) if hot is not None else NO_RESIDUAL
            g = Wg[e] @ x[t]
            u = Wu[e] @ x[t]
            if hrow != NO_RESIDUAL and "gate" in res:
                g = g + res["gate"][hrow] @ x[t]
                u = u + res["up"][hrow] @ x[t]
            h = swiglu(g, u, limit)
            if h_round == "bfloat16":
                h = round_bf16(h)
            elif h_round is not None:
                h = h.astype(h_round).astype(np.float64)
            y = Wd[e] @ h
            if hrow != NO_RESIDUAL and "down" in res:
                y = y + res["down"][hrow] @ h
            out[t] += w[t, j] * y
    return out


# --------------------------------------------------------------------------- route plan


def route_plan(rhs, num_experts: int, tile: int):
    """Token->expert gather plan (``vq_switch.py:100-152``).

    Returns ``order`` (stable sort of routes by expert), ``inverse`` (its
    inverse permutation), per-expert ``counts``/``offsets`` into the sorted
    routes and the tile descriptors ``(tile_expert, tile_offset, tile_count)``
    with at most ``tile`` routes per tile, tiles in expert order. Routes whose
    expert is outside ``[0, num_experts)`` sort after all others and their
    tiles come last, with expert ``-1``.
    """

    rhs = np.asarray(rhs).reshape(-1).astype(np.int64)
    key = np.where((rhs < 0) | (rhs >= num_experts), num_experts, rhs)  # invalid ids sort last
    order = np.argsort(key, kind="stable")
    inverse = np.empty_like(order)
    inverse[order] = np.arange(order.shape[0])
    allc = np.bincount(key, minlength=num_experts + 1)
    counts = allc[:num_experts]
    offsets = np.concatenate([[0], np.cumsum(counts)[:-1]])
    te, to, tc = [], [], []
    for e in range(num_experts + 1):  # the invalid routes' tiles last, with expert -1
        base = int(np.sum(allc[:e]))
        for start in range(0, int(allc[e]), tile):
            te.append(e if e < num_experts else -1)
            to.append(base + start)
            tc.append(min(tile, int(allc[e]) - start))
    return (order, inverse, counts, offsets,
            np.array(te, dtype=np.int64), np.array(to, dtype=np.int64), np.array(tc, dtype=np.int64))


# --------------------------------------------------------------------------- metrics


def max_rel_err(got, want) -> float:
    """``max |got - want| / max(|want|_inf, tiny)`` -- the normwise relative error."""

    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(want, dtype=np.float64)
    den = max(float(np.max(np.abs(r))) if r.size else 0.0, 1e-30)
    return float(np.max(np.abs(g - r))) / den if r.size else 0.0


def elementwise_ok(got, want, rtol=2e-3) -> bool:
    """Every element within ``rtol * max(|want_i|, rms(want))``."""

    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(want, dtype=np.float64)
    if r.size == 0:
        return True
    floor = float(np.sqrt(np.mean(r * r)))
    return bool(np.all(np.abs(g - r) <= rtol * np.maximum(np.abs(r), floor)))
