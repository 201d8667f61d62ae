"""The C-ABI library loads and exports every entry point ``include/keep_amd.h``
declares; host-only entry points and argument validation work without a GPU
(every validation error returns before any launch)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from keep_amd import _lib
from oracle import e8p

HEADER = Path(__file__).resolve().parents[1] / "include" / "keep_amd.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(keep_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in keep_amd.h but not exported"
    assert set(names) == set(_lib.EXPORTED)


def test_abi_version_and_empty_error():
    lib = _lib.load()
    assert lib.keep_abi_version() == 4
    # the 4 KiB int8 T / M tables, their check word, the 64 KiB LDS image
    assert lib.keep_e8p_prepared_bytes() == 4096 + 256 + 65536 == 69888
    assert isinstance(lib.keep_last_error(), bytes)


def test_host_codebooks_match_oracle():
    lib = _lib.load()
    out = (ctypes.c_uint32 * 256)()
    assert lib.keep_e8p_packed_abs_grid(out) == 0
    np.testing.assert_array_equal(np.frombuffer(out, dtype=np.uint32), e8p.e8p_packed_abs_grid())
    assert lib.keep_e8_1bit_packed(out) == 0
    np.testing.assert_array_equal(np.frombuffer(out, dtype=np.uint32), e8p.e8_1bit_packed())
    assert lib.keep_e8p_packed_abs_grid(None) == _lib.KEEP_EINVAL


def _matvec(**over):
    args = dict(x=16, x_dtype=1, x_rows=1, codes=16, code_bits=16, scales=16, scale_dtype=1, table=16, rhs=16, lhs=None,
                routes=1, x_div=1, E=1, N=16, K=64, gs=64, rc=None, rs=None, rgs=0, rt=None, hot=None, nhot=0,
                out=16, out_dtype=1, stream=None)
    args.update(over)
    return _lib.load().keep_vq_matvec(*args.values())


@pytest.mark.parametrize("over, msg", [
    (dict(code_bits=7), "code_bits"),
    (dict(K=60), "divisible by 8"),
    (dict(gs=24), "group_size"),
    (dict(x_dtype=9), "dtype"),
    (dict(x=None), "null"),
    (dict(x=3), "aligned"),
    (dict(rc=16, rs=None), "nested"),
    (dict(rhs=None, E=2), "rhs may be NULL only"),
])
def test_matvec_argument_validation_before_launch(over, msg):
    assert _matvec(**over) == _lib.KEEP_EINVAL
    assert msg in _lib.load().keep_last_error().decode()


def test_zero_routes_is_a_no_op():
    assert _matvec(routes=0, x=None) == 0


def test_other_entry_points_validate():
    lib = _lib.load()
    assert lib.keep_router_dual_topk(1, 1, 2000, 6, None, None, 0, 1, 1.0, 0.3, None, 0, 1, 1, None, None, None,
                                     None) == -1
    assert b"E must be" in lib.keep_last_error()
    assert lib.keep_route_plan(1, 10, 4, 4, 1, 1, 1, 1, 1, 1, 1, 2, 1, None) == -1
    assert b"max_tiles" in lib.keep_last_error()
    assert lib.keep_moe_decode(16, 1, 1, 4096, 2048, 1, 1, 6, 384, 16, 16, 16, 16, 16, 16, 1, 100, 2048, 16, None,
                               0.0, 16, 16, 1, None) == -1
    assert b"group_size_h" in lib.keep_last_error()
    assert lib.keep_e8p_decode(16, 10, 16, 16, 1, 3, 1, 16, None) == -1


def _tiles_layer(**over):
    args = dict(logits=16, bias_s=None, bias_d=None, func=0, renorm=1, route_scale=1.0, tau=0.3, slot_map=None,
                num_slots=0, E=384, k=6, x=16, x_dtype=1, T=8, H=4096, I=2048, gc=16, gs=16, uc=16, us=16, dc=16,
                ds=16, sdt=1, gsh=4096, gsi=2048, prep=16, limit=0.0, idx=16, w=16, want=None, want_score=None,
                admit=None, h_work=16, ws=256, ws_bytes=1 << 40, out=16, out_dtype=1, stream=None)
    args.update(over)
    return _lib.load().keep_moe_tiles_layer(*args.values())


@pytest.mark.parametrize("over, msg", [
    (dict(E=2000), "num_experts must be"),
    (dict(func=5), "score_func"),
    (dict(slot_map=16, num_slots=0), "num_slots"),
    (dict(k=17), "shape not served"),
    (dict(T=300), "shape not served"),
    (dict(x_dtype=3), "fp16 or bf16"),
    (dict(logits=None), "null pointer"),
    (dict(ws_bytes=1024), "workspace needs"),
])
def test_tiles_layer_argument_validation_before_launch(over, msg):
    assert _tiles_layer(**over) == _lib.KEEP_EINVAL
    assert msg in _lib.load().keep_last_error().decode()


def _nested_gemm(**over):
    args = dict(x=16, x_dtype=1, x_rows=4, lhs=None, oidx=None, codes=16, scales=16, sdt=1, prep=16, rc=16, rs=16,
                rsdt=1, hot=16, hot_rows=2, table=16, te=16, to=16, tc=16, n_tiles=1, routes=4, E=8, N=256, K=512,
                ws=256, ws_bytes=1 << 20, out=16, odt=0, stream=None)
    args.update(over)
    return _lib.load().keep_vq_grouped_gemm_nested_q8(*args.values())


@pytest.mark.parametrize("over, msg", [
    (dict(K=500), "multiple of 128"),
    (dict(hot=None), "null pointer"),
    (dict(rc=4), "8-byte aligned"),
    (dict(rsdt=7), "dtype enum"),
    (dict(x_dtype=2, ws=None), "workspace"),
])
def test_nested_gemm_argument_validation_before_launch(over, msg):
    assert _nested_gemm(**over) == _lib.KEEP_EINVAL
    assert msg in _lib.load().keep_last_error().decode()


def test_nested_swiglu_argument_validation_before_launch():
    lib = _lib.load()
    args = [16, 1, 4, None, 16, 16, 16, 16, 1, 16, 16, 16, 16, 16, 1, None, 2, 16, 16, 16, 16, 1, 4, 8, 256, 512,
            0.0, None, 0, 16, None]
    assert lib.keep_vq_grouped_swiglu_nested_q8(*args) == _lib.KEEP_EINVAL
    assert b"null pointer" in lib.keep_last_error()
