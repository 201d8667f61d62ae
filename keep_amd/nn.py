"""Module layer of the routed E8P expert path (torch, GPU).

- ``QuantizedVQLinear`` -- dense E8P/E8 linear (``src/ramp/nn/linear.py:17-121``).
- ``QuantizedVQSwitchLinear`` -- stacked E8P/E8 expert projection, drop-in for
  ``src/ramp/nn/switch_linear.py:93-463`` (core routing; the continuous
  sidecars -- scale delta, low-rank and sparse-row residuals, rotation
  matrices -- are outside this path and rejected with ``ValueError``).
- ``QuantizedVQSwitchGLU`` -- gate/up/down with SwiGLU, drop-in for
  ``src/ramp/models/glm4_moe_adapter.py:113-390``: few-token calls run the
  decode mat-vec per projection, prefill runs one device route plan shared by
  the three MFMA grouped GEMMs (``_shared_sorted_route_prefill``).
- ``LimitedSwiGLU`` -- ``deepseek_v4_flash_adapter.py:962-986``.
- ``RoutedVQMoE`` -- router + experts + weighted combine
  (``DeepseekV4FlashVQMoE.__call__``, ``deepseek_v4_flash_adapter.py:1776-1784``),
  whose decode path is the fused two-launch ``keep_moe_decode``.
"""

from __future__ import annotations

from typing import Callable

import numpy as np
import torch

from keep_amd import _lib, ops
from keep_amd.router import RouterOutput, _slot_args, router_dual_topk

CODEWORD_DIM = 8


class LimitedSwiGLU:
    """``silu(min(g, L)) * clip(u, -L, L)``; plain SwiGLU for ``L <= 0``.
    Called as ``act(up, gate)`` like the reference (``x`` first)."""

    def __init__(self, limit: float = 0.0, *, fp32: bool = False):
        self.limit = float(limit)
        self.fp32 = bool(fp32)

    def __call__(self, up: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        dtype = up.dtype
        g = gate.float() if self.fp32 else gate
        u = up.float() if self.fp32 else up
        if self.limit > 0:
            g = torch.clamp(g, max=self.limit)
            u = torch.clamp(u, -self.limit, self.limit)
        return (torch.nn.functional.silu(g) * u).to(dtype)


class QuantizedVQLinear:
    """Dense linear layer on E8 VQ codes (torch, GPU): ``vq_qmv`` for one row,
    ``vq_qmm`` for more, after the optional RHT or input rotation, plus bias
    (reference ``src/ramp/nn/linear.py:17-121``). ``x @ rotation_matrix`` runs
    in ``x``'s dtype, as ``apply_rotation_mx`` does (``keep/quant/rotation.py:39-43``)."""

    def __init__(self, *, input_dims: int, output_dims: int, codes, scales, codebook=None, bias=None,
                 group_size: int = 512, code_bits: int = 8, rht_signs=None, rotation_matrix=None):
        if input_dims <= 0 or output_dims <= 0:
            raise ValueError("input_dims and output_dims must be positive")
        if input_dims % CODEWORD_DIM != 0:
            raise ValueError("input_dims must be divisible by 8")
        if input_dims % group_size != 0:
            raise ValueError("input_dims must be divisible by group_size")
        if code_bits not in (8, 16):
            raise ValueError("code_bits must be 8 or 16")
        if tuple(codes.shape) != (output_dims, input_dims // CODEWORD_DIM):
            raise ValueError(f"codes must have shape ({output_dims}, {input_dims // CODEWORD_DIM}), "
                             f"found {tuple(codes.shape)}")
        if tuple(scales.shape) != (output_dims, input_dims // group_size):
            raise ValueError(f"scales must have shape ({output_dims}, {input_dims // group_size}), "
                             f"found {tuple(scales.shape)}")
        if bias is not None and tuple(bias.shape) != (output_dims,):
            raise ValueError(f"bias must have shape ({output_dims},), found {tuple(bias.shape)}")
        if rht_signs is not None and rotation_matrix is not None:
            raise ValueError("rht_signs and rotation_matrix are mutually exclusive")
        if rht_signs is not None and tuple(rht_signs.shape) != (input_dims,):
            raise ValueError(f"rht_signs must have shape ({input_dims},), found {tuple(rht_signs.shape)}")
        if rotation_matrix is not None and tuple(rotation_matrix.shape) != (input_dims, input_dims):
            raise ValueError(f"rotation_matrix must have shape ({input_dims}, {input_dims}), "
                             f"found {tuple(rotation_matrix.shape)}")
        device = codes.device if isinstance(codes, torch.Tensor) and codes.is_cuda else ops._device_of(codes)
        self.input_dims, self.output_dims = input_dims, output_dims
        self.group_size, self.code_bits = group_size, code_bits
        self.codes = ops._codes_tensor(codes, code_bits, device)
        self.scales = ops._to_dev(scales, device)
        self.codebook = ops._codebook_tensor(codebook, code_bits, device)
        self.bias = None if bias is None else ops._to_dev(bias, device)
        self.rht_signs = None if rht_signs is None else ops._to_dev(rht_signs, device, torch.float32)
        if self.rht_signs is not None:
            from keep_amd.rht import check_signs
            check_signs(self.rht_signs)
        self.rotation_matrix = None if rotation_matrix is None else ops._to_dev(rotation_matrix, device,
                                                                                torch.float32)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.input_dims:
            raise ValueError(f"input trailing dimension must be {self.input_dims}, found {x.shape[-1]}")
        if self.rht_signs is not None:
            from keep_amd.rht import apply_rht
            x = apply_rht(x, self.rht_signs, validate_signs=False)  # checked once, at construction
        if self.rotation_matrix is not None:
            x = x @ self.rotation_matrix.to(x.dtype)
        flat = x.reshape(-1, self.input_dims)
        kw = dict(in_dim=self.input_dims, out_dim=self.output_dims, group_size=self.group_size,
                  code_bits=self.code_bits)
        if flat.shape[0] == 1:
            y = ops.vq_qmv(flat[0], self.codes, self.scales, self.codebook, **kw).reshape(1, self.output_dims)
        else:
            y = ops.vq_qmm(flat, self.codes, self.scales, self.codebook, **kw)
        y = y.reshape(tuple(x.shape[:-1]) + (self.output_dims,))
        if self.bias is not None:
            y = y + self.bias  # type promotion as MLX's: a float32 bias gives a float32 result
        return y

    def _extra_repr(self) -> str:
        return f"{self.input_dims}, {self.output_dims}, group_size={self.group_size}, code_bits={self.code_bits}"

    @classmethod
    def from_weights(cls, weight, bias=None, *, group_size: int = 512, code_bits: int = 8, rht_signs=None,
                     rotation_matrix=None) -> "QuantizedVQLinear":
        """Quantise a dense ``[out, in]`` weight on the GPU (``linear.py:123-160``):
        the RHT (or rotation) is applied to the weight's rows as it will be to
        the inputs, then the data-free RTN (``encode.quantize_weight_rtn``)."""

        from keep_amd.encode import quantize_weight_rtn

        if rht_signs is not None and rotation_matrix is not None:
            raise ValueError("rht_signs and rotation_matrix are mutually exclusive")
        w = weight if isinstance(weight, torch.Tensor) else torch.from_numpy(np.asarray(weight, dtype=np.float32))
        device = w.device if w.is_cuda else torch.device("cuda", torch.cuda.current_device())
        w = w.to(device=device, dtype=torch.float32)
        if rht_signs is not None:
            from keep_amd.rht import apply_rht
            w = apply_rht(w, torch.as_tensor(rht_signs).to(device))
        if rotation_matrix is not None:
            w = w @ torch.as_tensor(rotation_matrix).to(device=device, dtype=torch.float32)
        q = quantize_weight_rtn(w, group_size=group_size, code_bits=code_bits)
        out_dim, in_dim = w.shape
        return cls(input_dims=in_dim, output_dims=out_dim, codes=q.codes, scales=q.scales,
                   codebook=torch.from_numpy(q.codebook.view(np.int32)).to(device), bias=bias,
                   group_size=q.group_size, code_bits=q.code_bits, rht_signs=rht_signs,
                   rotation_matrix=rotation_matrix)


class QuantizedVQSwitchLinear:
    """Switch-linear layer backed by stacked VQ expert tensors (torch, GPU)."""

    def __init__(self, *, input_dims: int, output_dims: int, num_experts: int, codes: torch.Tensor,
                 scales: torch.Tensor, codebook: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                 group_size: int = 512, code_bits: int = 8, use_gather_vqmm: bool = True,
                 route_strategy: str = "auto", gather_codebook_duplication: int = 8,
                 rht_signs: torch.Tensor | None = None, rotation_matrix: torch.Tensor | None = None, **sidecars):
        if input_dims <= 0 or output_dims <= 0 or num_experts <= 0:
            raise ValueError("input_dims, output_dims, and num_experts must be positive")
        if input_dims % CODEWORD_DIM != 0:
            raise ValueError("input_dims must be divisible by 8")
        if input_dims % group_size != 0:
            raise ValueError("input_dims must be divisible by group_size")
        if code_bits not in (8, 16):
            raise ValueError("code_bits must be 8 or 16")
        if gather_codebook_duplication not in (1, 4, 8):
            raise ValueError("gather_codebook_duplication must be 1, 4, or 8")
        if route_strategy not in ("auto", "direct", "sorted_tiled", "per_route_decoded"):
            raise ValueError("route_strategy must be 'auto', 'direct', 'sorted_tiled', or 'per_route_decoded'")
        unsupported = [k for k, v in sidecars.items() if v is not None]
        if unsupported:
            raise ValueError(f"continuous sidecars are not part of the routed E8P path: {sorted(unsupported)}")
        expected_codes = (num_experts, output_dims, input_dims // CODEWORD_DIM)
        expected_scales = (num_experts, output_dims, input_dims // group_size)
        if tuple(codes.shape) != expected_codes:
            raise ValueError(f"codes must have shape {expected_codes}, found {tuple(codes.shape)}")
        if tuple(scales.shape) != expected_scales:
            raise ValueError(f"scales must have shape {expected_scales}, found {tuple(scales.shape)}")
        if bias is not None and tuple(bias.shape) != (num_experts, output_dims):
            raise ValueError(f"bias must have shape ({num_experts}, {output_dims}), found {tuple(bias.shape)}")
        if rht_signs is not None and tuple(rht_signs.shape) != (input_dims,):
            raise ValueError(f"rht_signs must have shape ({input_dims},), found {tuple(rht_signs.shape)}")
        if rht_signs is not None and rotation_matrix is not None:
            raise ValueError("rht_signs and rotation_matrix are mutually exclusive")
        if rotation_matrix is not None and tuple(rotation_matrix.shape) != (input_dims, input_dims):
            raise ValueError(f"rotation_matrix must have shape ({input_dims}, {input_dims}), "
                             f"found {tuple(rotation_matrix.shape)}")
        device = codes.device if isinstance(codes, torch.Tensor) and codes.is_cuda else ops._device_of(codes)
        self.input_dims, self.output_dims, self.num_experts = input_dims, output_dims, num_experts
        self.group_size, self.code_bits = group_size, code_bits
        self.use_gather_vqmm, self.route_strategy = use_gather_vqmm, route_strategy
        self.gather_codebook_duplication = gather_codebook_duplication
        self.codes = ops._codes_tensor(codes, code_bits, device)
        self.scales = ops._to_dev(scales, device)
        self.codebook = ops._codebook_tensor(codebook, code_bits, device)
        self.bias = None if bias is None else ops._to_dev(bias, device)
        self.rht_signs = None if rht_signs is None else ops._to_dev(rht_signs, device, torch.float32)
        if self.rht_signs is not None:
            from keep_amd.rht import check_signs
            check_signs(self.rht_signs)
        self.rotation_matrix = None if rotation_matrix is None else ops._to_dev(rotation_matrix, device,
                                                                                torch.float32)

    @classmethod
    def from_weights(cls, weight, bias=None, *, group_size: int = 512, code_bits: int = 8,
                     use_gather_vqmm: bool = True, route_strategy: str = "auto",
                     gather_codebook_duplication: int = 8, rht_signs=None,
                     rotation_matrix=None) -> "QuantizedVQSwitchLinear":
        """Quantise stacked dense expert weights ``[E, out, in]`` on the GPU
        (``switch_linear.py:527-571``): the RHT (or rotation) of every expert's
        rows, as the inputs will get it, then each expert's data-free RTN. The
        RTN's scales belong to one (row, group), so the E experts quantise as one
        ``[E * out, in]`` matrix in a single pass."""

        from keep_amd.encode import quantize_weight_rtn

        if rht_signs is not None and rotation_matrix is not None:
            raise ValueError("rht_signs and rotation_matrix are mutually exclusive")
        w = weight if isinstance(weight, torch.Tensor) else torch.from_numpy(np.asarray(weight, dtype=np.float32))
        if w.ndim != 3:
            raise ValueError(f"weight must be 3D [experts, out, in], found {tuple(w.shape)}")
        device = w.device if w.is_cuda else torch.device("cuda", torch.cuda.current_device())
        w = w.to(device=device, dtype=torch.float32).contiguous()
        num_experts, out_dim, in_dim = w.shape
        if rht_signs is not None:
            from keep_amd.rht import apply_rht
            w = apply_rht(w, torch.as_tensor(rht_signs).to(device))
        if rotation_matrix is not None:
            w = w @ torch.as_tensor(rotation_matrix).to(device=device, dtype=torch.float32)
        q = quantize_weight_rtn(w.reshape(num_experts * out_dim, in_dim), group_size=group_size, code_bits=code_bits)
        return cls(input_dims=in_dim, output_dims=out_dim, num_experts=num_experts,
                   codes=q.codes.reshape(num_experts, out_dim, in_dim // CODEWORD_DIM),
                   scales=q.scales.reshape(num_experts, out_dim, in_dim // q.group_size),
                   codebook=torch.from_numpy(q.codebook.view(np.int32)).to(device), bias=bias,
                   group_size=q.group_size, code_bits=q.code_bits, use_gather_vqmm=use_gather_vqmm,
                   route_strategy=route_strategy, gather_codebook_duplication=gather_codebook_duplication,
                   rht_signs=None if rht_signs is None else torch.as_tensor(rht_signs).to(device),
                   rotation_matrix=None if rotation_matrix is None else torch.as_tensor(rotation_matrix))

    def effective_scales(self) -> torch.Tensor:
        return self.scales

    def _rht(self, x: torch.Tensor) -> torch.Tensor:
        """The input transform the weights were quantised under: RHT, or
        ``x @ rotation_matrix`` in ``x``'s dtype (``switch_linear.py:318-325``)."""
        if self.rotation_matrix is not None:
            return x @ self.rotation_matrix.to(x.dtype)
        if self.rht_signs is None:
            return x
        from keep_amd.rht import apply_rht
        return apply_rht(x, self.rht_signs, validate_signs=False)  # checked once, at construction

    def __call__(self, x: torch.Tensor, indices: torch.Tensor, *, sorted_indices: bool = False) -> torch.Tensor:
        x = self._rht(x)
        kw = dict(input_dims=self.input_dims, output_dims=self.output_dims, group_size=self.group_size,
                  code_bits=self.code_bits, route_strategy=self.route_strategy, sorted_indices=sorted_indices,
                  codebook_duplication=self.gather_codebook_duplication)
        if x.ndim >= 2 and indices.ndim >= 2 and tuple(x.shape[:-1]) == tuple(indices.shape[:-1]):
            lead, k = tuple(x.shape[:-1]), indices.shape[-1]
            y = ops.gather_vqmm(x.reshape(-1, self.input_dims), self.codes, self.scales, self.codebook,
                                indices.reshape(-1, k), **kw)
            y = y.reshape(lead + (k, self.output_dims))
        elif x.ndim >= 2 and tuple(x.shape[:-1]) == tuple(indices.shape):
            shape = tuple(indices.shape)
            flat_x = x.reshape(-1, self.input_dims)
            lhs = torch.arange(flat_x.shape[0], dtype=torch.int32, device=flat_x.device)
            y = ops.gather_vqmm(flat_x, self.codes, self.scales, self.codebook, indices.reshape(-1),
                                lhs_indices=lhs, **kw).reshape(shape + (self.output_dims,))
        else:
            raise ValueError(f"x {tuple(x.shape)} and indices {tuple(indices.shape)} match neither the token nor "
                             "the per-route layout")
        if self.bias is not None:
            y = y + self.bias[indices.long()].to(y.dtype)
        return y


class HotTier:
    """The nested 3-bit tier of a routed SwiGLU block: for the experts with a
    row in ``hot_of_slot`` (``uint32 [E]``, ``0xFFFFFFFF`` = none), an 8-bit E8
    residual per projection, ``residual[name] = (codes uint8 [H, N, K/8],
    scales [H, N, G])`` for ``name`` in gate / up / down, added to the E8P base
    (``e8p_nested_m1.py:90-112``; the serving step ``omlx_lattice.py:172-186,
    358-370``)."""

    def __init__(self, hot_of_slot, residual: dict):
        if set(residual) != {"gate", "up", "down"}:
            raise ValueError("the hot tier needs residual codes and scales for gate, up and down")
        dev = residual["gate"][0].device
        if not isinstance(hot_of_slot, torch.Tensor):
            hot_of_slot = torch.from_numpy(np.asarray(hot_of_slot, dtype=np.uint32).view(np.int32).copy())
        self.hot_of_slot = hot_of_slot.to(dev)
        self.residual_arrays = {n: (ops._codes_tensor(c, 8, dev), ops._to_dev(sc, dev))
                                for n, (c, sc) in residual.items()}
        self.rows = int(self.residual_arrays["gate"][0].shape[0])
        # every table form made here, so that no call copies from the host (graph capture)
        self._pairs = ops._to_dev(ops.e8_1bit_half2_table().view(np.int32), dev)
        self._table = ops._to_dev(ops.pair_packed(ops.e8_1bit_packed()).view(np.int32), dev)
        self._table_packed = ops._to_dev(ops.e8_1bit_packed().view(np.int32), dev)
        ops._unpaired_table(self._table)
        hot = self.hot_of_slot.to(torch.int64) & 0xFFFFFFFF
        self._hot32 = torch.where(hot == ops.NO_RESIDUAL, torch.full_like(hot, -1), hot).to(torch.int32)
        self._rows = self._hot32.cpu().numpy().astype(np.int64)  # host copy of the slot rows (-1: none)
        self._dirty = False
        self._image = None

    def route_slot(self, slot: int, row: int | None) -> None:
        """Pool row ``slot`` now holds an expert whose residual row is ``row``
        (None: an expert without one). The device rows change at the next
        ``publish()``, in the current stream's order, as a residency cache
        moves experts between slots (``omlx_lattice.py:274-278``)."""
        if not 0 <= slot < self._rows.size:
            raise ValueError(f"slot {slot} out of range for {self._rows.size} pool rows")
        if row is not None and not 0 <= row < self.rows:
            raise ValueError(f"residual row {row} out of range for a tier of {self.rows} rows")
        v = -1 if row is None else int(row)
        if self._rows[slot] != v:
            self._rows[slot], self._dirty = v, True

    def publish(self) -> None:
        """Queue the slot rows changed by ``route_slot`` on the current stream
        (pinned staging: the host may change them again at once)."""
        if not self._dirty:
            return
        rows = torch.from_numpy(self._rows.astype(np.int32)).pin_memory()
        self._hot32.copy_(rows, non_blocking=True)
        self.hot_of_slot.view(torch.int32).copy_(rows, non_blocking=True)  # -1 is NO_RESIDUAL's bits
        self._dirty = False

    def image(self) -> torch.Tensor:
        """The residual table's LDS image for the fused decode layer (built once, on the tier's device)."""
        if self._image is None:
            lib = _lib.load()
            img = torch.empty(lib.keep_e8_1bit_image_bytes(), dtype=torch.uint8, device=self._table_packed.device)
            _lib.call("keep_e8_1bit_image", self._table_packed.data_ptr(), img.data_ptr(),
                      ops._stream(img.device))
            self._image = img
        return self._image

    def layer_groups(self, hidden: int, intermediate: int):
        """``(group_size_h, group_size_i)`` of the residual scales, or None when
        the fused decode layer cannot take them (groups of 256-multiples)."""
        gh = hidden // self.residual_arrays["gate"][1].shape[-1]
        gi = intermediate // self.residual_arrays["down"][1].shape[-1]
        dts = {sc.dtype for _, sc in self.residual_arrays.values()}
        if self.residual_arrays["up"][1].shape[-1] != self.residual_arrays["gate"][1].shape[-1] or len(dts) != 1:
            return None
        if gh % 256 or gi % 256 or hidden % gh or intermediate % gi:
            return None
        return gh, gi

    def check(self, glu) -> None:
        hot = self.hot_of_slot
        if str(hot.dtype).rsplit(".", 1)[-1] not in ("uint32", "int32") or hot.numel() != glu.num_experts:
            raise ValueError(f"hot_of_slot must be uint32 [{glu.num_experts}]")
        for name, proj in (("gate", glu.gate_proj), ("up", glu.up_proj), ("down", glu.down_proj)):
            c, sc = self.residual_arrays[name]
            if c.ndim != 3 or tuple(c.shape[1:]) != (proj.output_dims, proj.input_dims // CODEWORD_DIM):
                raise ValueError(f"{name} residual codes must be [H, {proj.output_dims}, {proj.input_dims // 8}]")
            if sc.ndim != 3 or tuple(sc.shape[:2]) != tuple(c.shape[:2]):
                raise ValueError(f"{name} residual scales must be [H, {proj.output_dims}, groups]")

    def nested(self, name: str):
        """``(codes, scales, half2 table)`` for the one-pass nested mat-vec."""
        c, sc = self.residual_arrays[name]
        return c, sc, self._pairs

    def route_rows(self, rhs: torch.Tensor) -> torch.Tensor:
        """The residual row of every route (int32 bits; ``0xFFFFFFFF`` = none)."""
        hot = self.hot_of_slot.to(torch.int64) & 0xFFFFFFFF
        rows = hot[rhs.long().clamp(0, hot.numel() - 1)]
        rows = torch.where((rhs < 0) | (rhs >= hot.numel()), torch.full_like(rows, 0xFFFFFFFF), rows)
        return (rows - ((rows >> 31) << 32)).to(torch.int32)

    def residual(self, name: str, rows: torch.Tensor, route_rows: torch.Tensor) -> torch.Tensor:
        """Per-route residual ``[R, N]`` of routes ``rows[r]`` at residual rows
        ``route_rows[r]`` (zeros off the tier)."""
        c, sc = self.residual_arrays[name]
        return ops.e8_1bit_m1_per_route(rows, c, sc, self._table, route_rows, output_dims=c.shape[1])


class QuantizedVQSwitchGLU:
    """Routed SwiGLU experts: ``down(act(up(x), gate(x)))`` per route -> ``[..., k, H]``."""

    def __init__(self, *, gate_proj: QuantizedVQSwitchLinear, up_proj: QuantizedVQSwitchLinear,
                 down_proj: QuantizedVQSwitchLinear, prefill_engine: str = "auto",
                 activation: Callable | None = None, hot_tier: HotTier | None = None):
        if gate_proj.input_dims != up_proj.input_dims:
            raise ValueError("gate_proj and up_proj input dimensions must match")
        if gate_proj.output_dims != up_proj.output_dims:
            raise ValueError("gate_proj and up_proj output dimensions must match")
        if down_proj.input_dims != gate_proj.output_dims:
            raise ValueError("down_proj input dimension must match routed hidden dimension")
        if down_proj.output_dims != gate_proj.input_dims:
            raise ValueError("down_proj output dimension must match routed input dimension")
        if prefill_engine not in ("auto", "vq_metal", "nax_e8", "nax_e8p", "mfma"):
            raise ValueError("prefill_engine must be 'auto' or 'mfma'")
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj
        self.prefill_engine = prefill_engine
        self.activation = activation
        self.input_dims = gate_proj.input_dims
        self.hidden_dims = gate_proj.output_dims
        self.num_experts = gate_proj.num_experts
        if hot_tier is not None:
            hot_tier.check(self)
        self.hot_tier = hot_tier

    def _apply_activation(self, up: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        if self.activation is None:
            return torch.nn.functional.silu(gate) * up
        return self.activation(up, gate)

    def _all_e8p(self) -> bool:
        return all(p.code_bits == 16 and p.bias is None and p.rht_signs is None and p.rotation_matrix is None
                   for p in (self.gate_proj, self.up_proj, self.down_proj))

    def _can_use_shared_sorted_route_prefill(self, x: torch.Tensor, indices: torch.Tensor) -> bool:
        routes = indices.numel()
        return (self._all_e8p() and routes >= ops.GEMM_ROUTE_THRESHOLD
                and all(ops.gemm_eligible(code_bits=16, x_dtype=x.dtype, input_dims=p.input_dims,
                                          group_size=p.group_size)
                        for p in (self.gate_proj, self.up_proj, self.down_proj)))

    def _fused_swiglu_limit(self) -> float | None:
        """The SwiGLU limit when the activation is one the gate/up kernel
        applies itself (plain or limited SwiGLU in fp32), else None."""

        if self.activation is None:
            return 0.0
        if isinstance(self.activation, LimitedSwiGLU):
            return self.activation.limit
        return None

    def _nested_prefill_fused(self, limit: float | None) -> bool:
        """Whether the tiered prefill runs on the fused base-plus-residual
        kernels: a fused SwiGLU, one scale per row for every base and residual
        projection, gate and up scales (and their residuals') of one dtype."""

        ht, g, u, d = self.hot_tier, self.gate_proj, self.up_proj, self.down_proj
        if limit is None or g.scales.dtype != u.scales.dtype:
            return False
        if any(p.group_size != p.input_dims for p in (g, u, d)):
            return False
        res = [ht.residual_arrays[n][1] for n in ("gate", "up", "down")]
        return all(sc.shape[-1] == 1 for sc in res) and res[0].dtype == res[1].dtype

    def _shared_sorted_route_prefill(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """One device route plan shared by gate, up and down
        (``glm4_moe_adapter.py:274-353``): gate and up in one grouped GEMM
        with SwiGLU in its epilogue (h in bf16), down scattered straight back
        to route order; per-route outputs are float32."""
        lead, k = tuple(x.shape[:-1]), indices.shape[-1]
        flat_x = x.reshape(-1, self.input_dims).contiguous()
        flat_rhs = indices.reshape(-1).to(torch.int32).contiguous()
        R = flat_rhs.numel()
        order, inverse, _, _, te, to, tc, _ = ops.route_plan(flat_rhs, self.num_experts, ops.GEMM_ROUTE_TILE)
        sorted_lhs = torch.div(order, k, rounding_mode="floor")  # route r is token r // k's
        tiles = (te, to, tc)
        g, u, d = self.gate_proj, self.up_proj, self.down_proj
        f32 = torch.float32
        limit = self._fused_swiglu_limit()
        ht = self.hot_tier
        if ht is not None and self._nested_prefill_fused(limit):
            # base and residual in one pass per kernel: a hot expert's tiles add its residual row before
            # the SwiGLU (gate/up) and before the store (down)
            rg, ru, rd = (ht.residual_arrays[n] for n in ("gate", "up", "down"))
            hidden = ops.grouped_swiglu_nested(flat_x, g.codes, g.scales, u.codes, u.scales, g.codebook, rg, ru,
                                               ht._hot32, ht._table_packed, tiles, lhs=sorted_lhs, routes=R,
                                               input_dims=g.input_dims, hidden_dims=g.output_dims, limit=limit)
            y = ops.grouped_gemm_nested(hidden, d.codes, d.scales, d.codebook, rd, ht._hot32, ht._table_packed, tiles,
                                        lhs=None, routes=R, input_dims=d.input_dims, output_dims=d.output_dims,
                                        out_dtype=f32, out_index=order)
            return y.reshape(lead + (k, d.output_dims))
        if ht is not None:  # base GEMMs, then the residual GEMMs over tiles of routes grouped by residual row
            rrows = ht.route_rows(flat_rhs)
            r_order, _, _, _, rte, rto, rtc, _ = ops.route_plan(rrows, ht.rows, ops.GEMM_ROUTE_TILE)
            ro = r_order.long()
            r_tiles = (rte, rto, rtc)
            at_base = inverse[ro].to(torch.int32).contiguous()  # each residual position's base output row
            gate = ops.grouped_gemm(flat_x, g.codes, g.scales, g.codebook, tiles, lhs=sorted_lhs, routes=R,
                                    input_dims=g.input_dims, output_dims=g.output_dims, group_size=g.group_size,
                                    out_dtype=f32)
            up = ops.grouped_gemm(flat_x, u.codes, u.scales, u.codebook, tiles, lhs=sorted_lhs, routes=R,
                                  input_dims=u.input_dims, output_dims=u.output_dims, group_size=u.group_size,
                                  out_dtype=f32)
            x_lhs = torch.div(r_order, k, rounding_mode="floor")
            for out_t, name, proj in ((gate, "gate", g), (up, "up", u)):
                rc, rs = ht.residual_arrays[name]
                ops.grouped_residual_add(out_t, flat_x, rc, rs, r_tiles, lhs=x_lhs, out_index=at_base, routes=R,
                                         input_dims=proj.input_dims, output_dims=proj.output_dims,
                                         group_size=proj.input_dims // rs.shape[-1], table=ht._table_packed)
            hidden = self._apply_activation(up, gate).to(torch.bfloat16).contiguous()
            y = ops.grouped_gemm(hidden, d.codes, d.scales, d.codebook, tiles, lhs=None, routes=R,
                                 input_dims=d.input_dims, output_dims=d.output_dims, group_size=d.group_size,
                                 out_dtype=f32, out_index=order)
            rc, rs = ht.residual_arrays["down"]
            ops.grouped_residual_add(y, hidden, rc, rs, r_tiles, lhs=at_base, out_index=r_order, routes=R,
                                     input_dims=d.input_dims, output_dims=d.output_dims,
                                     group_size=d.input_dims // rs.shape[-1], table=ht._table_packed)
            return y.reshape(lead + (k, d.output_dims))
        if limit is not None and g.group_size == u.group_size and g.scales.dtype == u.scales.dtype:
            hidden = ops.grouped_swiglu(flat_x, g.codes, g.scales, u.codes, u.scales, g.codebook, tiles,
                                        lhs=sorted_lhs, routes=R, input_dims=g.input_dims,
                                        hidden_dims=g.output_dims, group_size=g.group_size, limit=limit)
        else:
            gate = ops.grouped_gemm(flat_x, g.codes, g.scales, g.codebook, tiles, lhs=sorted_lhs, routes=R,
                                    input_dims=g.input_dims, output_dims=g.output_dims, group_size=g.group_size,
                                    out_dtype=f32)
            up = ops.grouped_gemm(flat_x, u.codes, u.scales, u.codebook, tiles, lhs=sorted_lhs, routes=R,
                                  input_dims=u.input_dims, output_dims=u.output_dims, group_size=u.group_size,
                                  out_dtype=f32)
            # activation in fp32, hidden held in bf16 (fp16 would overflow the SwiGLU product)
            hidden = self._apply_activation(up, gate).to(torch.bfloat16).contiguous()
        y = ops.grouped_gemm(hidden, d.codes, d.scales, d.codebook, tiles, lhs=None, routes=R,
                             input_dims=d.input_dims, output_dims=d.output_dims, group_size=d.group_size,
                             out_dtype=f32, out_index=order)
        return y.reshape(lead + (k, d.output_dims))

    def _nested_decode(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """Few routes with a hot tier: one pass over base and residual per
        projection (``omlx_lattice.py:358-370``): gate/up in the token layout,
        down per route on the bf16 hidden, every output in fp32."""
        ht, g, u, d = self.hot_tier, self.gate_proj, self.up_proj, self.down_proj
        lead, k = tuple(x.shape[:-1]), indices.shape[-1]
        rows = x.reshape(-1, self.input_dims).contiguous()
        idx = indices.reshape(-1).to(torch.int32).contiguous()
        f32 = torch.float32

        def nested(rows_, proj, name, x_div):
            rc, rs, rt = ht.nested(name)
            return ops.routed_matvec(rows_, proj.codes, proj.scales, proj.codebook, idx, x_div=x_div,
                                     input_dims=proj.input_dims, output_dims=proj.output_dims,
                                     group_size=proj.group_size, residual=(rc, rs, rt), hot_of_slot=ht._hot32,
                                     out_dtype=f32)

        gate = nested(rows, g, "gate", k)
        up = nested(rows, u, "up", k)
        h = self._apply_activation(up, gate).to(torch.bfloat16).contiguous()
        y = nested(h, d, "down", 1)
        return y.reshape(lead + (k, d.output_dims))

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        if self._can_use_shared_sorted_route_prefill(x, indices):
            return self._shared_sorted_route_prefill(x, indices)
        if self.hot_tier is not None:
            return self._nested_decode(x, indices)
        gate = self.gate_proj(x, indices)
        up = self.up_proj(x, indices)
        return self.down_proj(self._apply_activation(up, gate), indices)


def moe_decode(x: torch.Tensor, idx: torch.Tensor, weight: torch.Tensor, gate, up, down, *, limit: float = 0.0,
               codebook: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
               h_work: torch.Tensor | None = None, prepared: bool = True) -> torch.Tensor:
    """Fused routed SwiGLU MoE for few tokens: ``keep_moe_tiles`` (routes grouped
    per expert, each hit expert read once, on the int8 matrix cores; five
    launches) where it serves the shape, else ``keep_moe_decode`` (two launches
    of the packed-table kernels, any shape).

    ``gate``/``up``/``down`` are ``(codes, scales)``: gate/up ``[E, I, H/8]``,
    down ``[E, H, I/8]``. ``out[t] = sum_j w[t,j] * down_e(swiglu(gate_e x_t, up_e x_t))``
    with fp32 accumulation; h is held in bf16 and the routed sum is returned in
    float32 by default, as the reference's decode step keeps them
    (``scripts/v41_build/omlx_lattice.py:368-371``). ``prepared=False`` forces the
    packed-table kernels.
    """

    device = x.device
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("moe_decode needs float16 or bfloat16 activations")
    (gc, gs), (uc, us), (dc, ds) = gate, up, down
    E, I, Hc = gc.shape
    H = Hc * 8
    if x.ndim != 2 or x.shape[1] != H:
        raise ValueError(f"x must be [tokens, {H}], found {tuple(x.shape)}")
    if tuple(uc.shape) != (E, I, Hc) or tuple(dc.shape) != (E, H, I // 8):
        raise ValueError("gate/up codes must be [E, I, H/8] and down codes [E, H, I/8]")
    if not (gs.dtype == us.dtype == ds.dtype):
        raise ValueError("gate/up/down scales must share a dtype")
    T, k = idx.shape
    cb = ops._codebook_tensor(codebook, 16, device)
    od = out_dtype or torch.float32
    out = torch.empty((T, H), dtype=od, device=device)
    if h_work is None:
        h_work = torch.empty((T * k * I,), dtype=torch.bfloat16, device=device)
    elif h_work.numel() < T * k * I or h_work.dtype != torch.bfloat16:
        raise ValueError("h_work must hold T*k*I bfloat16 elements")
    idx32 = idx.to(torch.int32).contiguous()
    w32 = weight.to(torch.float32).contiguous()
    prep = ops.prepared_table(cb) if prepared else None
    gh, gi = H // gs.shape[-1], I // ds.shape[-1]
    if prep is not None and moe_tiles_supported(T, E, H, I, k, gh, gi):
        ws = torch.empty(int(_lib.load().keep_moe_tiles_workspace_bytes(T, k, E, H)), dtype=torch.uint8,
                         device=device)
        _lib.call("keep_moe_tiles", x.data_ptr(), ops._DT[x.dtype], T, H, I, idx32.data_ptr(), w32.data_ptr(), k, E,
                  gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), dc.data_ptr(), ds.data_ptr(),
                  ops._DT[gs.dtype], gh, gi, prep.data_ptr(), float(limit), h_work.data_ptr(), ws.data_ptr(),
                  ws.numel(), out.data_ptr(), ops._DT[od], ops._stream(device))
        return out
    _lib.call("keep_moe_decode", x.data_ptr(), ops._DT[x.dtype], T, H, I, idx32.data_ptr(), w32.data_ptr(), k, E,
              gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), dc.data_ptr(), ds.data_ptr(),
              ops._DT[gs.dtype], H // gs.shape[-1], I // ds.shape[-1], cb.data_ptr(), ops._ptr(prep),
              float(limit), h_work.data_ptr(), out.data_ptr(), ops._DT[od], ops._stream(device))
    return out


def moe_tiles_layer(x: torch.Tensor, logits: torch.Tensor, gate, up, down, *, k: int, bias_served=None,
                    bias_demand=None, score_func: str = "softmax", renormalize: bool = True,
                    route_scale: float = 1.0, tau: float = float("inf"), limit: float = 0.0,
                    codebook: torch.Tensor | None = None, out_dtype: torch.dtype | None = None, slot_map=None,
                    h_work: torch.Tensor | None = None):
    """A few tokens' whole MoE layer from the router logits (``keep_moe_tiles_layer``):
    ``router_dual_topk``'s outputs and ``moe_decode``'s result on the tiles path, byte
    for byte: up to 128 routes (``T * k``) over at most 512 experts the gate/up launch
    routes and plans itself (three launches), otherwise the router, the activation
    terms and the route plan run in one launch before it for up to 32 tokens.
    ``x [T, H]`` (fp16/bf16), ``logits [T, E]``; ``slot_map`` as
    in ``moe_layer``. Returns ``(out [T, H], RouterOutput)``; float32 by default."""

    device = x.device
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("moe_tiles_layer needs float16 or bfloat16 activations")
    if score_func not in _lib.SCORE_FUNCS:
        raise ValueError(f"score_func must be one of {sorted(_lib.SCORE_FUNCS)}")
    (gc, gs), (uc, us), (dc, ds) = gate, up, down
    S, I, Hc = gc.shape
    H = Hc * 8
    if x.ndim != 2 or x.shape[1] != H:
        raise ValueError(f"x must be [tokens, {H}], found {tuple(x.shape)}")
    if tuple(uc.shape) != (S, I, Hc) or tuple(dc.shape) != (S, H, I // 8):
        raise ValueError("gate/up codes must be [E, I, H/8] and down codes [E, H, I/8]")
    if not (gs.dtype == us.dtype == ds.dtype):
        raise ValueError("gate/up/down scales must share a dtype")
    T = x.shape[0]
    z = logits.to(device=device, dtype=torch.float32).reshape(T, -1).contiguous()
    E = z.shape[1]
    if slot_map is None and E != S:
        raise ValueError(f"logits must hold {S} experts, found {E}")
    sm, ns = _slot_args(slot_map, S if slot_map is not None else None, E, device)
    bs = None if bias_served is None else bias_served.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    bd = None if bias_demand is None else bias_demand.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if bias_demand is bias_served:
        bd = bs
    for name, b in (("bias_served", bs), ("bias_demand", bd)):
        if b is not None and b.numel() != E:
            raise ValueError(f"{name} must have {E} entries, found {b.numel()}")
    i32 = dict(dtype=torch.int32, device=device)
    f32 = dict(dtype=torch.float32, device=device)
    r = RouterOutput(torch.empty((T, k), **i32), torch.empty((T, k), **f32), torch.empty((T, k), **i32),
                     torch.empty((T, k), **f32), torch.empty((T, k), dtype=torch.uint8, device=device))
    od = out_dtype or torch.float32
    out = torch.empty((T, H), dtype=od, device=device)
    if h_work is None:
        h_work = torch.empty((T * k * I,), dtype=torch.bfloat16, device=device)
    elif h_work.numel() < T * k * I or h_work.dtype != torch.bfloat16:
        raise ValueError("h_work must hold T*k*I bfloat16 elements")
    cb = ops._codebook_tensor(codebook, 16, device)
    prep = ops.prepared_table(cb)
    gh, gi = H // gs.shape[-1], I // ds.shape[-1]
    ws = torch.empty(int(_lib.load().keep_moe_tiles_workspace_bytes(T, k, S, H)), dtype=torch.uint8, device=device)
    _lib.call("keep_moe_tiles_layer", z.data_ptr(), ops._ptr(bs), ops._ptr(bd), _lib.SCORE_FUNCS[score_func],
              int(bool(renormalize)), float(route_scale), float(tau), ops._ptr(sm), ns, E, k, x.data_ptr(),
              ops._DT[x.dtype], T, H, I, gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), dc.data_ptr(),
              ds.data_ptr(), ops._DT[gs.dtype], gh, gi, prep.data_ptr(), float(limit), r.idx.data_ptr(),
              r.weight.data_ptr(), r.want.data_ptr(), r.want_score.data_ptr(), r.admit.data_ptr(), h_work.data_ptr(),
              ws.data_ptr(), ws.numel(), out.data_ptr(), ops._DT[od], ops._stream(device))
    return out, r


def moe_tiles_supported(T: int, num_experts: int, hidden: int, intermediate: int, k: int, group_size_h: int,
                        group_size_i: int) -> bool:
    """Whether the expert-grouped few-token path (``keep_moe_tiles``) serves this shape."""

    return bool(_lib.load().keep_moe_tiles_supported(T, num_experts, hidden, intermediate, k, group_size_h,
                                                      group_size_i))


def moe_layer_supported(num_experts: int, hidden: int, intermediate: int, k: int, group_size_h: int,
                        group_size_i: int) -> bool:
    """Whether ``moe_layer`` (the two-launch routed decode layer) serves this shape."""

    return bool(_lib.load().keep_moe_layer_supported(num_experts, hidden, intermediate, k, group_size_h,
                                                     group_size_i))


_LAYER_WS: dict = {}


def layer_workspace(device: torch.device, k: int, intermediate: int) -> torch.Tensor:
    """The one-launch layer's workspace for ``device`` and the current stream:
    zero-filled once, then reused by every call on that stream (it carries the
    call counter that tags the exchanged SwiGLU outputs)."""

    need = int(_lib.load().keep_moe_layer1_workspace_bytes(k, intermediate))
    key = (str(device), torch.cuda.current_stream(device).cuda_stream)
    ws = _LAYER_WS.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=device)
        _LAYER_WS[key] = ws
    return ws


def layer_status(workspace: torch.Tensor) -> int:
    """Status word of a one-launch layer workspace (value 1: a wait gave up; value 2: a block's
    certified early routes differed from the exact selection, never expected)."""

    out = (_lib.c_uint32 * 1)()
    _lib.call("keep_moe_layer1_status", workspace.data_ptr(), out, ops._stream(workspace.device))
    return int(out[0])


def layer_spin_ticks(ticks: int) -> int:
    """Set the give-up budget of every later one-launch layer call in this
    process, in ticks of the GPU's 100 MHz real-time counter (default 20000:
    200 us); returns the previous budget. A call whose wait for another
    block's SwiGLU output outlasts it returns NaN for the routes that wait
    held and sets bit 1 of ``layer_status`` (zero the workspace before the
    next call)."""

    prev = (_lib.c_uint32 * 1)()
    _lib.call("keep_moe_layer1_set_spin_ticks", int(ticks), prev)
    return int(prev[0])


def _one_launch_ok(device: torch.device, E: int, H: int, I: int, k: int) -> bool:
    props = torch.cuda.get_device_properties(device)
    return (props.multi_processor_count >= 256 and H == 4096 and I in (512, 1024, 1536, 2048) and 1 <= k <= 8
            and k <= E <= 1024)


def moe_layer(x: torch.Tensor, logits: torch.Tensor, gate, up, down, *, k: int, bias_served=None, bias_demand=None,
              score_func: str = "softmax", renormalize: bool = True, route_scale: float = 1.0,
              tau: float = float("inf"), limit: float = 0.0, codebook: torch.Tensor | None = None,
              out_dtype: torch.dtype | None = None, h_work: torch.Tensor | None = None,
              hot_tier: HotTier | None = None, one_launch: bool = False,
              workspace: torch.Tensor | None = None, slot_map=None):
    """One token's whole MoE layer in two launches (``keep_moe_layer``): the dual
    top-k router (as ``router_dual_topk``) fused with gate/up/SwiGLU, then down +
    weighted combine. ``x [1, H]`` (fp16/bf16), ``logits [1, E]``. With
    ``hot_tier`` (``keep_moe_layer_nested``) the routes of experts on the
    nested tier add their 8-bit E8 residual to all three projections. With
    ``one_launch`` (``keep_moe_layer1``, with ``hot_tier``
    ``keep_moe_layer1_nested``) the same layer runs as one launch of 256
    co-resident blocks that pass h through ``workspace`` (by default
    ``layer_workspace(device, k, I)`` of the current stream); it serves
    H = 4096, I in {512, 1024, 1536, 2048}, k <= 8. With
    ``slot_map`` (int32 ``[E]``, expert -> pool row) the pools hold fewer rows
    than the router has experts (a residency cache's slots); ``RouterOutput.idx``
    then holds rows. Returns ``(out [1, H], RouterOutput)``; the output is
    float32 by default."""

    device = x.device
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("moe_layer needs float16 or bfloat16 activations")
    if score_func not in _lib.SCORE_FUNCS:
        raise ValueError(f"score_func must be one of {sorted(_lib.SCORE_FUNCS)}")
    (gc, gs), (uc, us), (dc, ds) = gate, up, down
    E, I, Hc = gc.shape
    H = Hc * 8
    if x.ndim != 2 or tuple(x.shape) != (1, H):
        raise ValueError(f"x must be [1, {H}], found {tuple(x.shape)}")
    if tuple(uc.shape) != (E, I, Hc) or tuple(dc.shape) != (E, H, I // 8):
        raise ValueError("gate/up codes must be [E, I, H/8] and down codes [E, H, I/8]")
    if not (gs.dtype == us.dtype == ds.dtype):
        raise ValueError("gate/up/down scales must share a dtype")
    z = logits.to(device=device, dtype=torch.float32).reshape(1, -1).contiguous()
    S = E  # pool rows
    if slot_map is not None:
        E = z.shape[1]
    elif z.shape[1] != E:
        raise ValueError(f"logits must hold {E} experts, found {z.shape[1]}")
    sm, ns = _slot_args(slot_map, S if slot_map is not None else None, E, device)
    gh, gi = H // gs.shape[-1], I // ds.shape[-1]
    if not one_launch and not moe_layer_supported(E, H, I, k, gh, gi):
        raise ValueError("shape not served by the routed decode layer; use router_dual_topk + moe_decode")
    bs = None if bias_served is None else bias_served.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    bd = None if bias_demand is None else bias_demand.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if bias_demand is bias_served:
        bd = bs
    for name, b in (("bias_served", bs), ("bias_demand", bd)):
        if b is not None and b.numel() != E:
            raise ValueError(f"{name} must have {E} entries, found {b.numel()}")
    i32 = dict(dtype=torch.int32, device=device)
    f32 = dict(dtype=torch.float32, device=device)
    r = RouterOutput(torch.empty((1, k), **i32), torch.empty((1, k), **f32), torch.empty((1, k), **i32),
                     torch.empty((1, k), **f32), torch.empty((1, k), dtype=torch.uint8, device=device))
    od = out_dtype or torch.float32
    out = torch.empty((1, H), dtype=od, device=device)
    cb = ops._codebook_tensor(codebook, 16, device)
    prep = ops.prepared_table(cb)
    if one_launch:
        if not _one_launch_ok(device, E, H, I, k):
            raise ValueError("shape or device not served by the one-launch layer (H = 4096, I in {512, 1024, 1536, "
                             "2048}, k <= 8, E <= 1024, 256 compute units)")
        need = int(_lib.load().keep_moe_layer1_workspace_bytes(k, I))
        ws = layer_workspace(device, k, I) if workspace is None else workspace
        if ws.dtype != torch.uint8 or ws.device != device or ws.numel() < need or not ws.is_contiguous():
            raise ValueError(f"workspace must be a contiguous uint8 tensor of at least {need} bytes on {device}")
        if hot_tier is not None:
            if hot_tier.hot_of_slot.numel() != S:
                raise ValueError(f"hot_of_slot must have {S} entries (one per pool row)")
            groups = hot_tier.layer_groups(H, I)
            if groups is None:
                raise ValueError("residual scale groups must be 256-element multiples (one dtype) for the decode layer")
            (rgc, rgs), (ruc, rus), (rdc, rds) = (hot_tier.residual_arrays[n] for n in ("gate", "up", "down"))
            _lib.call("keep_moe_layer1_nested", z.data_ptr(), ops._ptr(bs), ops._ptr(bd), _lib.SCORE_FUNCS[score_func],
                      int(bool(renormalize)), float(route_scale), float(tau), ops._ptr(sm), ns, E, k, x.data_ptr(),
                      ops._DT[x.dtype], H, I, gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(),
                      dc.data_ptr(), ds.data_ptr(), ops._DT[gs.dtype], gh, gi, prep.data_ptr(), float(limit),
                      r.idx.data_ptr(), r.weight.data_ptr(), r.want.data_ptr(), r.want_score.data_ptr(),
                      r.admit.data_ptr(), ws.data_ptr(), ws.numel(), out.data_ptr(), ops._DT[od],
                      hot_tier._hot32.data_ptr(), hot_tier.rows, rgc.data_ptr(), rgs.data_ptr(), ruc.data_ptr(),
                      rus.data_ptr(), rdc.data_ptr(), rds.data_ptr(), ops._DT[rgs.dtype], groups[0], groups[1],
                      hot_tier._table_packed.data_ptr(), ops._stream(device))
            return out, r
        _lib.call("keep_moe_layer1", z.data_ptr(), ops._ptr(bs), ops._ptr(bd), _lib.SCORE_FUNCS[score_func],
                  int(bool(renormalize)), float(route_scale), float(tau), ops._ptr(sm), ns, E, k, x.data_ptr(),
                  ops._DT[x.dtype], H, I, gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), dc.data_ptr(),
                  ds.data_ptr(), ops._DT[gs.dtype], gh, gi, prep.data_ptr(), float(limit), r.idx.data_ptr(),
                  r.weight.data_ptr(),
                  r.want.data_ptr(), r.want_score.data_ptr(), r.admit.data_ptr(), ws.data_ptr(), ws.numel(),
                  out.data_ptr(), ops._DT[od], ops._stream(device))
        return out, r
    if h_work is None:
        h_work = torch.empty((k * I,), dtype=torch.bfloat16, device=device)
    elif h_work.numel() < k * I or h_work.dtype != torch.bfloat16:
        raise ValueError("h_work must hold k*I bfloat16 elements")
    if hot_tier is not None:
        if hot_tier.hot_of_slot.numel() != S:
            raise ValueError(f"hot_of_slot must have {S} entries (one per pool row)")
        groups = hot_tier.layer_groups(H, I)
        if groups is None:
            raise ValueError("residual scale groups must be 256-element multiples (one dtype) for the decode layer")
        (rgc, rgs), (ruc, rus), (rdc, rds) = (hot_tier.residual_arrays[n] for n in ("gate", "up", "down"))
        hot_route = torch.empty((k,), **i32)
        _lib.call("keep_moe_layer_nested", z.data_ptr(), ops._ptr(bs), ops._ptr(bd), _lib.SCORE_FUNCS[score_func],
                  int(bool(renormalize)), float(route_scale), float(tau), ops._ptr(sm), ns, E, k, x.data_ptr(),
                  ops._DT[x.dtype], H, I, gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), dc.data_ptr(),
                  ds.data_ptr(), ops._DT[gs.dtype], gh, gi, prep.data_ptr(), float(limit), r.idx.data_ptr(),
                  r.weight.data_ptr(),
                  r.want.data_ptr(), r.want_score.data_ptr(), r.admit.data_ptr(), h_work.data_ptr(), out.data_ptr(),
                  ops._DT[od], hot_tier._hot32.data_ptr(), hot_tier.rows, rgc.data_ptr(), rgs.data_ptr(),
                  ruc.data_ptr(), rus.data_ptr(), rdc.data_ptr(), rds.data_ptr(), ops._DT[rgs.dtype], groups[0],
                  groups[1], hot_tier.image().data_ptr(), hot_route.data_ptr(), ops._stream(device))
        return out, r
    _lib.call("keep_moe_layer", z.data_ptr(), ops._ptr(bs), ops._ptr(bd), _lib.SCORE_FUNCS[score_func],
              int(bool(renormalize)), float(route_scale), float(tau), ops._ptr(sm), ns, E, k, x.data_ptr(),
              ops._DT[x.dtype], H, I, gc.data_ptr(), gs.data_ptr(), uc.data_ptr(), us.data_ptr(), dc.data_ptr(),
              ds.data_ptr(), ops._DT[gs.dtype], gh, gi, prep.data_ptr(), float(limit), r.idx.data_ptr(),
              r.weight.data_ptr(), r.want.data_ptr(), r.want_score.data_ptr(), r.admit.data_ptr(), h_work.data_ptr(),
              out.data_ptr(), ops._DT[od], ops._stream(device))
    return out, r


class RoutedVQMoE:
    """Router + routed E8P SwiGLU experts + weighted combine (one MoE layer).

    ``__call__(x, logits)`` evaluates the residency-biased dual top-k router
    once, then runs the experts: the fused decode pair for few tokens, the
    shared-plan MFMA path for prefill. Returns ``(out [T, H], RouterOutput)``.

    ``slot_map`` (int32 ``[E]``, expert -> row of ``glu``'s pools, e.g. a
    ``ResidencyCache``'s, with its ``bias_served``) serves a pool smaller than
    the router's ``num_experts``; ``RouterOutput.idx`` then holds pool rows.

    ``shared_experts`` (a one-expert ``QuantizedVQSwitchGLU``, every token on
    expert 0 with weight 1) adds the shared expert to the routed sum, and
    ``__call__(..., residual=h)`` adds the residual stream, both in fp32 and
    rounded once to ``out_dtype`` (``DeepseekV4FlashVQMoE.__call__``,
    ``deepseek_v4_flash_adapter.py:1777-1784``; ``omlx_lattice.py:374-388``).

    One token runs the fused two-launch layer (``keep_moe_layer``, or
    ``keep_moe_layer_nested`` with a hot tier). ``one_launch=True`` runs it as
    the one-launch layer where that serves the shape (``keep_moe_layer1`` /
    ``keep_moe_layer1_nested``, the current stream's ``layer_workspace``):
    faster, but it assumes all 256 of its blocks are resident together, so a
    caller sharing the GPU with other work checks ``layer_status`` for a wait
    that gave up (NaN output).
    """

    def __init__(self, glu: QuantizedVQSwitchGLU, *, top_k: int, score_func: str = "softmax",
                 renormalize: bool = True, route_scale: float = 1.0, swiglu_limit: float = 0.0,
                 bias_served: torch.Tensor | None = None, bias_demand: torch.Tensor | None = None,
                 tau: float = float("inf"), decode_max_tokens: int = 64, out_dtype=torch.float32,
                 shared_experts: QuantizedVQSwitchGLU | None = None, slot_map: torch.Tensor | None = None,
                 one_launch: bool = False):
        self.glu, self.top_k, self.score_func = glu, top_k, score_func
        self.one_launch = bool(one_launch)
        self.renormalize, self.route_scale, self.limit = renormalize, route_scale, float(swiglu_limit)
        self.bias_served, self.bias_demand, self.tau = bias_served, bias_demand, tau
        self.decode_max_tokens = decode_max_tokens
        self.out_dtype = out_dtype
        if glu.activation is None and self.limit > 0:
            glu.activation = LimitedSwiGLU(self.limit)
        if shared_experts is not None:
            if shared_experts.num_experts != 1:
                raise ValueError("shared_experts must be a one-expert QuantizedVQSwitchGLU")
            if shared_experts.input_dims != glu.input_dims:
                raise ValueError("shared_experts input dimension must match the routed experts'")
            if shared_experts.activation is None and self.limit > 0:
                shared_experts.activation = LimitedSwiGLU(self.limit)
        self.shared_experts = shared_experts
        self.slot_map = slot_map

    def shared(self, x: torch.Tensor) -> torch.Tensor:
        """The shared expert's output for every row of ``x``, float32 ``[T, H]``."""

        se = self.shared_experts
        T = x.shape[0]
        idx = torch.zeros((T, 1), dtype=torch.int32, device=x.device)
        w = torch.ones((T, 1), dtype=torch.float32, device=x.device)
        g, u, d = se.gate_proj, se.up_proj, se.down_proj
        if (T <= self.decode_max_tokens and se._all_e8p() and se.hot_tier is None
                and x.dtype in (torch.float16, torch.bfloat16)):
            return moe_decode(x, idx, w, (g.codes, g.scales), (u.codes, u.scales), (d.codes, d.scales),
                              limit=self.limit, codebook=g.codebook, out_dtype=torch.float32)
        return se(x, idx).reshape(T, -1).float()

    def experts(self, x: torch.Tensor, idx: torch.Tensor, weight: torch.Tensor, *,
                out_dtype: torch.dtype | None = None) -> torch.Tensor:
        g, u, d = self.glu.gate_proj, self.glu.up_proj, self.glu.down_proj
        od = out_dtype or self.out_dtype
        T = x.shape[0]
        if (T <= self.decode_max_tokens and self.glu._all_e8p() and self.glu.hot_tier is None
                and x.dtype in (torch.float16, torch.bfloat16)):
            return moe_decode(x, idx, weight, (g.codes, g.scales), (u.codes, u.scales), (d.codes, d.scales),
                              limit=self.limit, codebook=g.codebook, out_dtype=od)
        y = self.glu(x, idx)  # [T, k, H]
        return ops.route_combine(y, weight, od)

    def _layer_path(self, x: torch.Tensor) -> bool:
        g, d = self.glu.gate_proj, self.glu.down_proj
        ht = self.glu.hot_tier
        return (x.shape[0] == 1 and x.dtype in (torch.float16, torch.bfloat16) and self.glu._all_e8p() and
                (ht is None or ht.layer_groups(g.input_dims, g.output_dims) is not None) and
                self.decode_max_tokens >= 1 and
                moe_layer_supported(g.num_experts, g.input_dims, g.output_dims, self.top_k,
                                    g.input_dims // g.scales.shape[-1], d.input_dims // d.scales.shape[-1]))

    def _tiles_layer_path(self, x: torch.Tensor) -> bool:
        g, d = self.glu.gate_proj, self.glu.down_proj
        T = x.shape[0]
        return (2 <= T <= self.decode_max_tokens and x.dtype in (torch.float16, torch.bfloat16) and
                self.glu._all_e8p() and self.glu.hot_tier is None and self.top_k <= 16 and
                moe_tiles_supported(T, g.num_experts, g.input_dims, g.output_dims, self.top_k,
                                    g.input_dims // g.scales.shape[-1], d.input_dims // d.scales.shape[-1]))

    def __call__(self, x: torch.Tensor, logits: torch.Tensor, *, residual: torch.Tensor | None = None):
        extra = self.shared_experts is not None or residual is not None
        od = torch.float32 if extra else self.out_dtype
        if self._tiles_layer_path(x):
            g, u, d = self.glu.gate_proj, self.glu.up_proj, self.glu.down_proj
            out, r = moe_tiles_layer(x, logits, (g.codes, g.scales), (u.codes, u.scales), (d.codes, d.scales),
                                     k=self.top_k, bias_served=self.bias_served, bias_demand=self.bias_demand,
                                     score_func=self.score_func, renormalize=self.renormalize,
                                     route_scale=self.route_scale, tau=self.tau, limit=self.limit,
                                     codebook=g.codebook, out_dtype=od, slot_map=self.slot_map)
        elif self._layer_path(x):
            g, u, d = self.glu.gate_proj, self.glu.up_proj, self.glu.down_proj
            one = self.one_launch and _one_launch_ok(x.device, logits.shape[-1], g.input_dims, g.output_dims,
                                                     self.top_k)
            out, r = moe_layer(x, logits, (g.codes, g.scales), (u.codes, u.scales), (d.codes, d.scales),
                               k=self.top_k, bias_served=self.bias_served, bias_demand=self.bias_demand,
                               score_func=self.score_func, renormalize=self.renormalize,
                               route_scale=self.route_scale, tau=self.tau, limit=self.limit, codebook=g.codebook,
                               out_dtype=od, hot_tier=self.glu.hot_tier, slot_map=self.slot_map, one_launch=one)
        else:
            r = router_dual_topk(logits, self.top_k, bias_served=self.bias_served, bias_demand=self.bias_demand,
                                 score_func=self.score_func, renormalize=self.renormalize,
                                 route_scale=self.route_scale, tau=self.tau, slot_map=self.slot_map,
                                 num_slots=self.glu.num_experts)
            out = self.experts(x, r.idx, r.weight, out_dtype=od)
        if not extra:
            return out, r
        from keep_amd.block import combine_add
        sh = self.shared(x) if self.shared_experts is not None else None
        return combine_add(out, sh, residual, self.out_dtype), r
