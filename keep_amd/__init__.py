"""keep_amd -- MI355X (gfx950) routed E8P expert path.

Python host code over torch device tensors calling hand-written HIP kernels
through the C ABI of ``libkeep_amd.so`` (``include/keep_amd.h``). No CPU
fallback: without the library every operator raises ``RuntimeError``.
"""

from keep_amd._lib import is_available
from keep_amd.block import combine_add, rmsnorm_quant_rht
from keep_amd.encode import (encode_e8_1bit_rtn, encode_e8p_rtn, encode_e8p_rtn_diagonal_hessian,
                             quantize_weight_rtn)
from keep_amd.nn import (HotTier, LimitedSwiGLU, QuantizedVQLinear, QuantizedVQSwitchGLU, QuantizedVQSwitchLinear,
                         RoutedVQMoE, moe_decode, moe_layer, moe_layer_supported, moe_tiles_layer)
from keep_amd.ops import (
    decode_e8p,
    decode_weight_matrix,
    e8_1bit_m1_per_route,
    e8_1bit_m1_token_layout,
    e8_1bit_packed,
    e8p_m1_per_route,
    e8p_m1_token_layout,
    e8p_nested_m1_per_route,
    e8p_nested_m1_token_layout,
    e8p_packed_abs_grid,
    gather_vqmm,
    gather_vqmm_sorted_routes,
    gather_vqmm_verify_rows,
    half2_pairs,
    pair_packed,
    route_plan,
    trace_gather_vqmm_calls,
    vq_qmm,
    vq_qmv,
)
from keep_amd.residency import ResidencyCache, ResidencyPolicy, residual_cache
from keep_amd.router import expert_select, resident_bias, router_dual_topk

__all__ = [
    "HotTier", "LimitedSwiGLU", "encode_e8_1bit_rtn", "encode_e8p_rtn", "encode_e8p_rtn_diagonal_hessian",
    "quantize_weight_rtn", "ResidencyCache", "ResidencyPolicy", "residual_cache", "combine_add", "rmsnorm_quant_rht", "QuantizedVQLinear", "QuantizedVQSwitchGLU", "QuantizedVQSwitchLinear", "RoutedVQMoE", "decode_e8p",
    "decode_weight_matrix", "e8_1bit_m1_per_route", "e8_1bit_m1_token_layout", "e8_1bit_packed", "e8p_m1_per_route",
    "e8p_m1_token_layout", "e8p_nested_m1_per_route", "e8p_nested_m1_token_layout", "e8p_packed_abs_grid",
    "expert_select", "gather_vqmm", "gather_vqmm_sorted_routes", "gather_vqmm_verify_rows", "half2_pairs",
    "is_available", "moe_decode", "moe_layer", "moe_layer_supported", "moe_tiles_layer", "pair_packed", "resident_bias", "route_plan",
    "router_dual_topk", "trace_gather_vqmm_calls", "vq_qmm", "vq_qmv",
]
