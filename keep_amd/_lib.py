"""ctypes binding of ``libkeep_amd.so`` (the C ABI in ``include/keep_amd.h``).

The library is loaded lazily from this package directory. There is no CPU
fallback: if the library is missing or fails to load, every GPU operator
raises ``RuntimeError`` naming the problem.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_uint32, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get("KEEP_AMD_LIB", Path(__file__).resolve().parent / "libkeep_amd.so"))

KEEP_F32, KEEP_F16, KEEP_BF16 = 0, 1, 2
KEEP_OK, KEEP_EINVAL, KEEP_ELAUNCH, KEEP_EUNSUPPORTED = 0, -1, -2, -3
SCORE_FUNCS = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}

# name -> argtypes (all return int unless listed in _RESTYPE)
_P = c_void_p
_SIGS = {
    "keep_last_error": [],
    "keep_abi_version": [],
    "keep_e8p_packed_abs_grid": [POINTER(c_uint32)],
    "keep_e8_1bit_packed": [POINTER(c_uint32)],
    "keep_e8p_decode": [_P, c_int64, _P, _P, c_int, c_int64, c_int64, _P, _P],
    "keep_e8_1bit_decode": [_P, c_int64, _P, _P, c_int, c_int64, c_int64, _P, _P],
    "keep_vq_encode": [_P, c_int64, c_int, _P, c_int, _P, _P, c_int64, _P, _P],
    "keep_group_absmax": [_P, c_int64, c_int64, c_float, _P, _P],
    "keep_vq_matvec": [_P, c_int, c_int64, _P, c_int, _P, c_int, _P, _P, _P, c_int64, c_int64, c_int64, c_int64,
                       c_int64, c_int64, _P, _P, c_int64, _P, _P, c_int64, _P, c_int, _P],
    "keep_vq_matvec_tiles": [_P, c_int, c_int64, _P, c_int, _P, c_int, _P, _P, c_int64, _P, _P, _P, c_int64, c_int64,
                             c_int64, c_int64, c_int64, c_int64, _P, c_int, _P],
    "keep_router_dual_topk": [_P, c_int64, c_int64, c_int64, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, _P,
                              _P, _P, _P, _P, _P],
    "keep_route_plan": [_P, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, _P],
    "keep_moe_decode": [_P, c_int, c_int64, c_int64, c_int64, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
                        c_int, c_int64, c_int64, _P, _P, c_float, _P, _P, c_int, _P],
    "keep_moe_tiles": [_P, c_int, c_int64, c_int64, c_int64, _P, _P, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int,
                       c_int64, c_int64, _P, c_float, _P, _P, c_int64, _P, c_int, _P],
    "keep_moe_tiles_workspace_bytes": [c_int64, c_int64, c_int64, c_int64],
    "keep_moe_tiles_layer": [_P, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, c_int64, c_int64, _P, c_int,
                             c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, _P, c_float,
                             _P, _P, _P, _P, _P, _P, _P, c_int64, _P, c_int, _P],
    "keep_vq_grouped_gemm_q8_workspace_bytes": [c_int64, c_int64],
    "keep_route_combine": [_P, _P, c_int64, c_int64, c_int64, _P, c_int, _P],
    "keep_rht": [_P, c_int, _P, c_int, c_int64, c_int64, _P, c_int, _P],
    "keep_rmsnorm_quant_rht": [_P, c_int, c_int64, c_int64, _P, c_int, c_float, c_int64, c_int, _P, _P, _P, c_int, _P],
    "keep_moe_combine_add": [_P, _P, c_int, _P, c_int, c_int64, _P, c_int, _P],
    "keep_e8_1bit_matvec": [_P, c_int, c_int64, _P, _P, c_int, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64,
                            c_int64, _P, c_int, _P],
    "keep_vq_grouped_gemm_q8": [_P, c_int, c_int64, _P, _P, _P, c_int, _P, c_int, _P, _P, _P, _P, c_int64, c_int64,
                                c_int64, c_int64, c_int64, c_int64, _P, c_int64, _P, c_int, _P],
    "keep_vq_grouped_swiglu_q8": [_P, c_int, c_int64, _P, _P, _P, _P, _P, c_int, _P, _P, _P, _P, c_int64, c_int64,
                                  c_int64, c_int64, c_int64, c_int64, c_float, _P, c_int64, _P, _P],
    "keep_vq_grouped_swiglu_nested_q8": [_P, c_int, c_int64, _P, _P, _P, _P, _P, c_int, _P, _P, _P, _P, _P, c_int,
                                         _P, c_int64, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64,
                                         c_float, _P, c_int64, _P, _P],
    "keep_vq_grouped_gemm_nested_q8": [_P, c_int, c_int64, _P, _P, _P, _P, c_int, _P, _P, _P, c_int, _P, c_int64, _P,
                                       _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P, c_int64, _P,
                                       c_int, _P],
    "keep_moe_tiles_supported": [c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64],
    "keep_moe_gateup": [_P, c_int, c_int64, c_int64, c_int64, _P, _P, c_int64, c_int64, _P, _P, _P, _P, c_int,
                        c_int64, _P, _P, c_float, _P, _P],
    "keep_moe_layer_supported": [c_int64, c_int64, c_int64, c_int64, c_int64, c_int64],
    "keep_moe_layer": [_P, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, c_int64, c_int64, _P, c_int, c_int64,
                       c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, _P, c_float, _P, _P, _P, _P, _P, _P,
                       _P, c_int, _P],
    "keep_moe_layer_noalloc": [_P, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, c_int64, c_int64, _P, c_int,
                               c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, _P, c_float, _P, _P,
                               _P, _P, _P, _P, c_int, _P],
    "keep_moe_layer1": [_P, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, c_int64, c_int64, _P, c_int, c_int64,
                        c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, _P, c_float, _P, _P, _P, _P, _P, _P,
                        c_int64, _P, c_int, _P],
    "keep_moe_layer1_nested": [_P, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, c_int64, c_int64, _P, c_int,
                               c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, _P, c_float, _P, _P,
                               _P, _P, _P, _P, c_int64, _P, c_int, _P, c_int64, _P, _P, _P, _P, _P, _P, c_int,
                               c_int64, c_int64, _P, _P],
    "keep_moe_layer1_workspace_bytes": [c_int64, c_int64],
    "keep_moe_layer1_status": [_P, _P, _P],
    "keep_moe_layer1_set_spin_ticks": [c_uint32, _P],
    "keep_moe_layer_nested": [_P, _P, _P, c_int, c_int, c_float, c_float, _P, c_int64, c_int64, c_int64, _P, c_int,
                              c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64, _P, c_float, _P, _P,
                              _P, _P, _P, _P, _P, c_int, _P, c_int64, _P, _P, _P, _P, _P, _P, c_int, c_int64, c_int64,
                              _P, _P, _P],
    "keep_e8_1bit_image": [_P, _P, _P],
    "keep_e8_1bit_image_bytes": [],
    "keep_moe_down": [c_int, c_int64, c_int64, c_int64, _P, _P, c_int64, c_int64, _P, _P, c_int, c_int64, _P, _P, _P,
                      _P, c_int, _P],
    "keep_e8p_prepare": [_P, _P, _P],
    "keep_e8p_prepared_bytes": [],
}
_RESTYPE = {"keep_last_error": c_char_p, "keep_moe_tiles_workspace_bytes": c_int64,
            "keep_moe_layer1_workspace_bytes": c_int64,
            "keep_vq_grouped_gemm_q8_workspace_bytes": c_int64}
EXPORTED = tuple(_SIGS)

_lib = None
_load_error: str | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise ``RuntimeError`` if unavailable."""

    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise RuntimeError(_load_error)
    if not LIB_PATH.exists():
        _load_error = (f"keep_amd HIP library not found at {LIB_PATH}; build it with "
                       "`python -c 'import __graft_entry__ as g; g.build()'` or `python keep_amd/build.py`")
        raise RuntimeError(_load_error)
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the host
        _load_error = f"failed to load {LIB_PATH}: {exc}"
        raise RuntimeError(_load_error) from exc
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, c_int)
    _lib = lib
    return lib


def is_available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def check(rc: int, what: str) -> None:
    """Map a status code to ``ValueError`` (bad arguments) or ``RuntimeError``."""

    if rc == KEEP_OK:
        return
    msg = load().keep_last_error().decode(errors="replace")
    if rc == KEEP_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
