"""GPU parity: E8P decode (bit-exact) and the routed decode mat-vec family
(within max relative error 2e-3 of the float64 oracle, fp32 accumulate)."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import synth
from oracle import e8p, ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
# A bf16-stored output adds its own rounding (at most 2**-9 relative) on top of
# the fp32-accumulation bound; fp32-output checks of the same kernels hold TOL.
TOL_BF16_OUT = TOL + 2.0 ** -9


def _t(a, dev):
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check(got, want, tol=TOL):
    g = got.float().cpu().numpy()
    err = ops.max_rel_err(g, want)
    assert err <= tol, f"max rel err {err:.3e}"
    assert ops.elementwise_ok(g, want, rtol=tol), "elementwise bound violated"
    return err


def test_decode_every_codeword_bit_exact(dev):
    codes = np.arange(1 << 16, dtype=np.uint16)
    got = keep_amd.decode_e8p(_t(codes, dev)).cpu().numpy()
    np.testing.assert_array_equal(got, e8p.e8p_full_grid())


@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("G", [1, 4])
def test_decode_weight_matrix_scaled_bit_exact(dev, sdt, G):
    codes, scales = synth.projection_np(3, 40, 256, group_size=256 // G, seed=G)
    s = torch.from_numpy(scales.astype(np.float32)).to(sdt)
    got = keep_amd.decode_weight_matrix(_t(codes, dev), s.to(dev), code_bits=16).cpu().numpy()
    want = e8p.decode_weight_matrix(codes, s.float().numpy(), code_bits=16)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
def test_vq_qmv_config1_shape(dev, xdt):
    K, N = 4096, 2048
    codes, scales = synth.projection_np(1, N, K, seed=11)
    x = synth.rht_activations(1, K, seed=12, device=dev, dtype=xdt)[0]
    y = keep_amd.vq_qmv(x, _t(codes[0], dev), _t(scales[0], dev), in_dim=K, out_dim=N, group_size=K, code_bits=16)
    assert y.dtype == xdt and y.shape == (N,)
    want = ops.qmv(x.float().cpu().numpy(), codes[0], scales[0])
    _check(y, want, TOL_BF16_OUT if xdt == torch.bfloat16 else TOL)
    # the fp32-accumulated result itself (fp32 output) holds 2e-3 for every activation dtype
    y32 = keep_amd.ops.routed_matvec(x.reshape(1, K), _t(codes, dev), _t(scales, dev),
                                     keep_amd.ops._default_codebook(16, dev),
                                     torch.zeros(1, dtype=torch.int32, device=dev), input_dims=K, output_dims=N,
                                     group_size=K, out_dtype=torch.float32)
    _check(y32[0], want)


@pytest.mark.parametrize("E,N,K,gs", [(4, 93, 768, 768), (3, 64, 512, 64), (5, 130, 256, 32), (2, 16, 2048, 512)])
def test_gather_token_and_per_route_layouts(dev, E, N, K, gs):
    codes, scales = synth.projection_np(E, N, K, group_size=gs, seed=N)
    rng = np.random.default_rng(K)
    T, k = 3, 2
    rhs = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    x = synth.rht_activations(T, K, seed=5, device=dev) if K & (K - 1) == 0 else \
        torch.from_numpy(rng.standard_normal((T, K)).astype(np.float16)).to(dev)
    xc = x.float().cpu().numpy()
    y = keep_amd.e8p_m1_token_layout(x, _t(codes, dev), _t(scales, dev), None, _t(rhs, dev), output_dims=N)
    assert y.shape == (T, k, N)
    _check(y, ops.gather_token(xc, codes, scales, rhs))
    xr = torch.from_numpy(rng.standard_normal((T * k, K)).astype(np.float16)).to(dev)
    y2 = keep_amd.e8p_m1_per_route(xr, _t(codes, dev), _t(scales, dev), None, _t(rhs.reshape(-1), dev),
                                   output_dims=N)
    _check(y2, ops.gather_routes(xr.float().cpu().numpy(), codes, scales, rhs.reshape(-1), np.arange(T * k)))


def test_gather_vqmm_direct_matches_oracle_and_traces(dev):
    E, N, K = 8, 256, 1024
    codes, scales = synth.projection_np(E, N, K, group_size=512, seed=3)
    x = synth.rht_activations(2, K, seed=4, device=dev)
    rhs = np.array([[1, 7, 3], [0, 7, 5]], dtype=np.int32)
    with keep_amd.trace_gather_vqmm_calls() as tr:
        y = keep_amd.gather_vqmm(x, _t(codes, dev), _t(scales, dev), None, _t(rhs, dev), input_dims=K,
                                 output_dims=N, group_size=512, code_bits=16)
    assert tr and tr[0]["strategy"] == "direct" and tr[0]["route_count"] == 6
    _check(y, ops.gather_token(x.float().cpu().numpy(), codes, scales, rhs))


def test_code_bits_8_table(dev):
    rng = np.random.default_rng(21)
    E, N, K = 3, 48, 512
    codes = rng.integers(0, 256, size=(E, N, K // 8), dtype=np.uint8)
    scales = np.exp(rng.normal(0, 0.3, size=(E, N, 2))).astype(np.float16)
    x = torch.from_numpy(rng.standard_normal((2, K)).astype(np.float16)).to(dev)
    rhs = np.array([[2, 0], [1, 1]], dtype=np.int32)
    y = keep_amd.gather_vqmm(x, _t(codes, dev), _t(scales, dev), None, _t(rhs, dev), input_dims=K, output_dims=N,
                             group_size=256, code_bits=8)
    want = ops.gather_token(x.float().cpu().numpy(), codes, scales, rhs, code_bits=8)
    _check(y, want)


def test_nested_residual_tier(dev):
    rng = np.random.default_rng(31)
    E, N, K, H = 6, 96, 512, 2
    codes, scales = synth.projection_np(E, N, K, seed=32)
    rcodes = rng.integers(0, 256, size=(H, N, K // 8), dtype=np.uint8)
    rscales = np.exp(rng.normal(-1.0, 0.3, size=(H, N, 1))).astype(np.float16)
    hot = np.full(E, ops.NO_RESIDUAL, dtype=np.uint32)
    hot[1], hot[4] = 0, 1
    table = keep_amd.ops.e8_1bit_half2_table()
    x = synth.rht_activations(1, K, seed=33, device=dev)
    rhs = np.array([[1, 2, 4]], dtype=np.int32)
    y = keep_amd.e8p_nested_m1_token_layout(x, (_t(codes, dev), _t(scales, dev), None), _t(rhs, dev),
                                            (_t(rcodes, dev), _t(rscales, dev), _t(table, dev)), _t(hot, dev),
                                            output_dims=N)
    want = ops.nested_routes(x.float().cpu().numpy(), (codes, scales), (rcodes, rscales), hot, rhs.reshape(-1),
                             np.zeros(3, dtype=np.int64)).reshape(1, 3, N)
    _check(y, want)
    # a base-tier route equals the plain kernel bit for bit
    plain = keep_amd.e8p_m1_token_layout(x, _t(codes, dev), _t(scales, dev), None, _t(rhs, dev), output_dims=N)
    assert torch.equal(plain[0, 1], y[0, 1])


def test_out_of_range_route_gives_nan_row_not_fault(dev):
    codes, scales = synth.projection_np(2, 32, 256, seed=1)
    x = synth.rht_activations(1, 256, seed=2, device=dev)
    rhs = torch.tensor([[0, 5]], dtype=torch.int32, device=dev)
    y = keep_amd.e8p_m1_token_layout(x, _t(codes, dev), _t(scales, dev), None, rhs, output_dims=32)
    assert torch.isfinite(y[0, 0]).all() and torch.isnan(y[0, 1]).all()
    with pytest.raises(ValueError, match="rhs_indices must be in"):
        keep_amd.gather_vqmm(x, _t(codes, dev), _t(scales, dev), None, rhs, input_dims=256, output_dims=32,
                             group_size=256, code_bits=16, validate_indices=True)


def test_vq_qmm_rows(dev):
    K, N, M = 1024, 200, 5
    codes, scales = synth.projection_np(1, N, K, group_size=256, seed=8)
    x = torch.from_numpy(np.random.default_rng(9).standard_normal((M, K)).astype(np.float32)).to(dev)
    y = keep_amd.vq_qmm(x, _t(codes[0], dev), _t(scales[0], dev), in_dim=K, out_dim=N, group_size=256, code_bits=16)
    _check(y, ops.qmm(x.cpu().numpy(), codes[0], scales[0]))
