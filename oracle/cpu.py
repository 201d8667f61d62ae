"""ctypes loader of ``oracle/libkeep_oracle.so`` (``cpu_ref.c``) -- test
infrastructure and the timed CPU baseline; never used by ``keep_amd``."""

from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libkeep_oracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        lib.oracle_e8p_decode.argtypes = [c_void_p, c_int64, c_void_p, c_void_p]
        lib.oracle_e8p_decode.restype = None
        lib.oracle_routed_matvec.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                             c_int64, c_int64, c_int64, c_int64, c_void_p, c_int]
        lib.oracle_routed_matvec.restype = None
        lib.oracle_routed_matvec8.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                              c_int64, c_int64, c_int64, c_int64, c_void_p, c_int]
        lib.oracle_routed_matvec8.restype = None
        lib.oracle_moe_decode.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                          c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                          c_int64, c_void_p, c_float, c_int, c_void_p, c_int]
        lib.oracle_moe_decode.restype = None
        lib.oracle_moe_decode_nested.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                                 c_int64, c_void_p, c_float, c_int, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
                                                 c_void_p, c_int]
        lib.oracle_moe_decode_nested.restype = None
        lib.oracle_nearest.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p]
        lib.oracle_nearest.restype = None
        lib.oracle_max_threads.restype = c_int
        _lib = lib
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def max_threads() -> int:
    return int(load().oracle_max_threads())


def decode(codes: np.ndarray, table: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint16).reshape(-1)
    t = np.ascontiguousarray(table, dtype=np.uint32)
    out = np.empty((c.size, 8), dtype=np.float32)
    load().oracle_e8p_decode(_p(c), c.size, _p(t), _p(out))
    return out.reshape(np.shape(codes) + (8,))


def routed_matvec(x, codes, scales, table, rhs, lhs=None, *, x_div=1, group_size, threads=0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.uint16)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    t = np.ascontiguousarray(table, dtype=np.uint32)
    rhs = np.ascontiguousarray(rhs, dtype=np.int32).reshape(-1)
    lhs = None if lhs is None else np.ascontiguousarray(lhs, dtype=np.int32).reshape(-1)
    E, N, C = codes.shape
    out = np.empty((rhs.size, N), dtype=np.float32)
    load().oracle_routed_matvec(_p(x), _p(codes), _p(scales), _p(t), _p(rhs), _p(lhs), rhs.size, x_div, N, C * 8,
                                group_size, _p(out), int(threads))
    return out


def routed_matvec8(x, codes, scales, table8, rhs, lhs=None, *, x_div=1, group_size, threads=0) -> np.ndarray:
    """The nested tier's residual projection per route: rows ``rhs[r]`` of the
    8-bit E8 codes ``[nhot, N, K/8]`` (``rhs[r] < 0``: zeros), the same fp32
    row dot as ``moe_decode_nested``'s residual."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    t8 = np.ascontiguousarray(table8, dtype=np.uint32)
    rhs = np.ascontiguousarray(rhs, dtype=np.int32).reshape(-1)
    lhs = None if lhs is None else np.ascontiguousarray(lhs, dtype=np.int32).reshape(-1)
    _, N, C = codes.shape
    out = np.empty((rhs.size, N), dtype=np.float32)
    load().oracle_routed_matvec8(_p(x), _p(codes), _p(scales), _p(t8), _p(rhs), _p(lhs), rhs.size, x_div, N, C * 8,
                                 group_size, _p(out), int(threads))
    return out


def moe_decode(x, idx, w, gate, up, down, table, *, limit=0.0, h_bf16=True, threads=0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    (gc, gs), (uc, us), (dc, ds) = [(np.ascontiguousarray(c, dtype=np.uint16), np.ascontiguousarray(s, np.float32))
                                    for c, s in (gate, up, down)]
    t = np.ascontiguousarray(table, dtype=np.uint32)
    T, H = x.shape
    k = idx.shape[1]
    I = gc.shape[1]
    out = np.empty((T, H), dtype=np.float32)
    load().oracle_moe_decode(_p(x), T, H, I, _p(idx), _p(w), k, _p(gc), _p(gs), _p(uc), _p(us), _p(dc), _p(ds),
                             H // gs.shape[-1], I // ds.shape[-1], _p(t), float(limit), int(bool(h_bf16)), _p(out),
                             int(threads))
    return out


def moe_decode_nested(x, idx, w, gate, up, down, table, hot_of_slot, residual, table8, *, limit=0.0, h_bf16=True,
                      threads=0) -> np.ndarray:
    """``moe_decode`` with the nested tier: ``hot_of_slot[e]`` is expert e's row in
    ``residual[name] = (uint8 codes [nhot, N, K/8], scales [nhot, N, G])`` or
    ``0xFFFFFFFF`` (none); ``table8`` is the packed 8-bit E8 table."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    (gc, gs), (uc, us), (dc, ds) = [(np.ascontiguousarray(c, dtype=np.uint16), np.ascontiguousarray(s, np.float32))
                                    for c, s in (gate, up, down)]
    (rgc, rgs), (ruc, rus), (rdc, rds) = [(np.ascontiguousarray(residual[n][0], dtype=np.uint8),
                                           np.ascontiguousarray(residual[n][1], dtype=np.float32))
                                          for n in ("gate", "up", "down")]
    hot = np.asarray(hot_of_slot, dtype=np.uint32).astype(np.int64)
    hot = np.ascontiguousarray(np.where(hot == 0xFFFFFFFF, -1, hot), dtype=np.int32)
    t = np.ascontiguousarray(table, dtype=np.uint32)
    t8 = np.ascontiguousarray(table8, dtype=np.uint32)
    T, H = x.shape
    k = idx.shape[1]
    I = gc.shape[1]
    out = np.empty((T, H), dtype=np.float32)
    load().oracle_moe_decode_nested(_p(x), T, H, I, _p(idx), _p(w), k, _p(gc), _p(gs), _p(uc), _p(us), _p(dc),
                                    _p(ds), H // gs.shape[-1], I // ds.shape[-1], _p(t), float(limit),
                                    int(bool(h_bf16)), _p(hot), _p(rgc), _p(rgs), _p(ruc), _p(rus), _p(rdc), _p(rds),
                                    H // rgs.shape[-1], I // rds.shape[-1], _p(t8), _p(out), int(threads))
    return out


def nearest(vectors, grid, w=None) -> np.ndarray:
    """Exhaustive weighted nearest codeword (``oracle_nearest``): ``w`` None,
    ``[8]`` (shared) or ``[n, 8]``; ties to the lowest grid index."""

    v = np.ascontiguousarray(vectors, dtype=np.float32).reshape(-1, 8)
    g = np.ascontiguousarray(grid, dtype=np.float32).reshape(-1, 8)
    out = np.empty(v.shape[0], dtype=np.int64)
    stride = 0
    wa = None
    if w is not None:
        wa = np.ascontiguousarray(w, dtype=np.float32)
        stride = 0 if wa.ndim == 1 else 8
        if wa.size not in (8, v.size):
            raise ValueError("w must be [8] or [n, 8]")
    load().oracle_nearest(_p(v), v.shape[0], _p(wa), stride, _p(g), g.shape[0], _p(out))
    return out
