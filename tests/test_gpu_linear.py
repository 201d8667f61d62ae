"""GPU parity of the dense VQ layer (QuantizedVQLinear, reference
src/ramp/nn/linear.py:17-121) and of the 8-bit E8 dense decode
(decode_weight_matrix(code_bits=8), reference src/keep/vq/e8.py:542-571):
the decode bit-exact against the oracle's, the layer within 2e-3 of the
float64 oracle (oracle RHT / rotation, dense decode, bias)."""

import numpy as np
import pytest
import torch

import keep_amd
from oracle import e8p, ops
from oracle import rht as orht

pytestmark = pytest.mark.gpu
TOL = 2e-3
OUT_TOL = {torch.float32: TOL, torch.float16: TOL + 2.0 ** -11, torch.bfloat16: TOL + 2.0 ** -9}


def _check(got, want, tol=TOL):
    g = got.float().cpu().numpy()
    err = ops.max_rel_err(g, want)
    assert err <= tol, f"max rel err {err:.3e}"
    assert ops.elementwise_ok(g, want, rtol=tol), "elementwise bound violated"
    return err


def test_decode_weight_matrix_8bit_every_code_bit_exact(dev):
    codes = np.arange(256, dtype=np.uint8).reshape(4, 64)
    got = keep_amd.decode_weight_matrix(torch.from_numpy(codes).to(dev)).cpu().numpy()  # code_bits defaults to 8
    np.testing.assert_array_equal(got, e8p.decode_weight_matrix(codes, code_bits=8))
    np.testing.assert_array_equal(got.reshape(256, 8), e8p.decode_e8_1bit(np.arange(256, dtype=np.uint8)))


@pytest.mark.parametrize("sdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("G", [1, 4])
def test_decode_weight_matrix_8bit_scaled_bit_exact(dev, sdt, G):
    rng = np.random.default_rng(G)
    codes = rng.integers(0, 256, size=(3, 40, 32), dtype=np.uint8)
    s = torch.from_numpy(np.exp(rng.normal(0, 0.3, size=(3, 40, G))).astype(np.float32)).to(sdt)
    got = keep_amd.decode_weight_matrix(torch.from_numpy(codes).to(dev), s.to(dev), code_bits=8).cpu().numpy()
    np.testing.assert_array_equal(got, e8p.decode_weight_matrix(codes, s.float().numpy(), code_bits=8))


def _layer(dev, N, K, G, code_bits, seed, *, bias=False, rht=False, rotation=False):
    rng = np.random.default_rng(seed)
    if code_bits == 16:
        codes = rng.integers(0, 1 << 16, size=(N, K // 8), dtype=np.uint16)
        ct = torch.from_numpy(codes.view(np.int16)).to(dev)
    else:
        codes = rng.integers(0, 256, size=(N, K // 8), dtype=np.uint8)
        ct = torch.from_numpy(codes).to(dev)
    scales = np.exp(rng.normal(0, 0.3, size=(N, K // G))).astype(np.float16)
    b = rng.normal(0, 1, size=N).astype(np.float32) if bias else None
    signs = np.where(rng.integers(0, 2, size=K) == 1, 1.0, -1.0).astype(np.float32) if rht else None
    R = np.linalg.qr(rng.normal(size=(K, K)))[0].astype(np.float32) if rotation else None
    layer = keep_amd.QuantizedVQLinear(
        input_dims=K, output_dims=N, codes=ct, scales=torch.from_numpy(scales).to(dev),
        bias=None if b is None else torch.from_numpy(b).to(dev), group_size=G, code_bits=code_bits,
        rht_signs=None if signs is None else torch.from_numpy(signs).to(dev),
        rotation_matrix=None if R is None else torch.from_numpy(R).to(dev))
    W = ops.dense(codes, scales.astype(np.float32), code_bits=code_bits)

    def want(x):
        xf = x.float().cpu().numpy().astype(np.float64).reshape(-1, K)
        if signs is not None:
            xf = orht.apply_rht(xf, signs)
        if R is not None:
            xf = xf @ R.astype(np.float64)
        y = xf @ W.T
        if b is not None:
            y = y + b
        return y.reshape(tuple(x.shape[:-1]) + (N,))
    return layer, want


@pytest.mark.parametrize("code_bits", [8, 16])
@pytest.mark.parametrize("lead,xdt", [((1,), torch.float16), ((5,), torch.bfloat16), ((2, 3), torch.float32),
                                      ((), torch.float16)])
def test_quantized_vq_linear_vs_oracle(dev, code_bits, lead, xdt):
    N, K, G = 160, 1024, 512
    layer, want = _layer(dev, N, K, G, code_bits, seed=code_bits + len(lead), bias=True)
    x = torch.from_numpy(np.random.default_rng(7).standard_normal(lead + (K,)).astype(np.float32)).to(xdt).to(dev)
    y = layer(x)
    assert y.shape == lead + (N,) and y.dtype == torch.float32  # a float32 bias promotes, as in MLX
    _check(y, want(x), OUT_TOL[xdt])


@pytest.mark.parametrize("mode", ["rht", "rotation"])
@pytest.mark.parametrize("M", [1, 4])
def test_quantized_vq_linear_input_transforms(dev, mode, M):
    """The RHT (or an orthogonal input rotation) is applied to x before the
    codes, as the reference layer does; rotation runs in x's dtype, so fp32
    activations keep the 2e-3 bound."""
    N, K, G = 96, 512, 256
    layer, want = _layer(dev, N, K, G, 16, seed=M, rht=mode == "rht", rotation=mode == "rotation")
    xdt = torch.float16 if mode == "rht" else torch.float32
    x = torch.from_numpy(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32)).to(xdt).to(dev)
    _check(layer(x), want(x), OUT_TOL[xdt] + (2.0 ** -11 if mode == "rht" else 0.0))


def test_quantized_vq_linear_rejects_bad_shapes(dev):
    c = torch.zeros((16, 64), dtype=torch.uint8, device=dev)
    s = torch.ones((16, 1), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="codes must have shape"):
        keep_amd.QuantizedVQLinear(input_dims=256, output_dims=16, codes=c, scales=s, group_size=256)
    with pytest.raises(ValueError, match="mutually exclusive"):
        keep_amd.QuantizedVQLinear(input_dims=512, output_dims=16, codes=c, scales=s, group_size=512,
                                   rht_signs=torch.ones(512, device=dev), rotation_matrix=torch.eye(512, device=dev))
    layer = keep_amd.QuantizedVQLinear(input_dims=512, output_dims=16, codes=c, scales=s, group_size=512)
    with pytest.raises(ValueError, match="trailing dimension"):
        layer(torch.zeros((2, 256), dtype=torch.float16, device=dev))
