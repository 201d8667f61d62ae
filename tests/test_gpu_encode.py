"""GPU encoders against the exhaustive scan of the C oracle (oracle/encode.py):
the factored E8P search and the 8-bit E8 scan bit for bit, unweighted, with
one shared diagonal and with one per vector, on random vectors, on every
codeword, on exact ties (midpoints of neighbouring codewords), on targets of
exactly zero and on zero weights (free signs: the lowest code); the RTN
quantiser's codes and fp16 scales bit for bit; QuantizedVQLinear.from_weights
with the RHT applied to the weight rows."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import encode as kenc
from oracle import e8p
from oracle import encode as oenc
from oracle import rht as orht

pytestmark = pytest.mark.gpu


def _u(codes):
    c = codes.cpu().numpy()
    return c.view(np.uint16) if c.dtype == np.int16 else c


@pytest.mark.parametrize("code_bits", [8, 16])
def test_every_codeword_encodes_to_itself(dev, code_bits):
    g = oenc.grid(code_bits)
    enc = kenc.encode_e8p_rtn if code_bits == 16 else kenc.encode_e8_1bit_rtn
    np.testing.assert_array_equal(_u(enc(torch.from_numpy(g).to(dev))), np.arange(len(g)))
    if code_bits == 16:
        w = np.abs(np.random.default_rng(1).standard_normal(8)).astype(np.float32) + 0.05
        np.testing.assert_array_equal(_u(kenc.encode_e8p_rtn_diagonal_hessian(g, w)), np.arange(len(g)))


@pytest.mark.parametrize("mode", ["none", "unit", "shared", "per_row"])
def test_e8p_random_vectors_bit_exact(dev, mode):
    rng = np.random.default_rng(20260711)
    v = (rng.standard_normal((6000, 8)) * 0.6).astype(np.float32)
    if mode == "none":
        got, w = kenc.encode_e8p_rtn(v), None
    elif mode == "unit":
        w = np.ones(8, np.float32)
        got = kenc.encode_e8p_rtn_diagonal_hessian(v, w)
        np.testing.assert_array_equal(_u(got), _u(kenc.encode_e8p_rtn(v)))  # unit diagonal = unweighted
    elif mode == "shared":
        w = np.abs(rng.standard_normal(8)).astype(np.float32) + 0.05
        got = kenc.encode_e8p_rtn_diagonal_hessian(v, w)
        np.testing.assert_array_equal(_u(got), _u(kenc.encode_e8p_rtn_diagonal_hessian(v, np.broadcast_to(w, v.shape))))
    else:
        w = np.abs(rng.standard_normal((6000, 8))).astype(np.float32) + 0.05
        got = kenc.encode_e8p_rtn_diagonal_hessian(v, w)
    np.testing.assert_array_equal(_u(got), oenc.nearest(v, 16, w))


@pytest.mark.parametrize("code_bits", [8, 16])
def test_ties_zero_targets_and_zero_weights(dev, code_bits):
    g = oenc.grid(code_bits)
    rng = np.random.default_rng(101)
    m = min(2000, len(g) - 1)
    mid = ((g[:m] + g[1:m + 1]) / 2).astype(np.float32)  # exact ties under unit weights
    quarter = (rng.integers(-12, 13, (1000, 8)) / 4).astype(np.float32)  # targets of exactly zero after a shift
    for v, w in ((mid, None), (quarter, None), (quarter, np.array([1, 1, 0, 1, 2, 0, 1, 3], np.float32)),
                 (mid, np.array([0, 1, 1, 1, 1, 1, 1, 0], np.float32))):
        enc = (kenc.encode_e8p_rtn if w is None else lambda a: kenc.encode_e8p_rtn_diagonal_hessian(a, w)) \
            if code_bits == 16 else None
        if code_bits == 8:
            if w is not None:
                continue
            got = kenc.encode_e8_1bit_rtn(v)
        else:
            got = enc(v)
        np.testing.assert_array_equal(_u(got), oenc.nearest(v, code_bits, w))


def test_e8_1bit_random_bit_exact(dev):
    v = (np.random.default_rng(3).standard_normal((20000, 8)) * 1.5).astype(np.float32)
    got = kenc.encode_e8_1bit_rtn(torch.from_numpy(v).to(dev))
    assert got.dtype == torch.uint8
    np.testing.assert_array_equal(_u(got), oenc.nearest(v, 8))


@pytest.mark.parametrize("code_bits,group", [(16, 512), (16, 64), (8, 128)])
def test_quantize_weight_rtn_bit_exact(dev, code_bits, group):
    rng = np.random.default_rng(code_bits + group)
    w = (rng.standard_normal((96, 1024)) * 0.04).astype(np.float32)
    w[3, :group] = 0.0  # a zero group: scale 0, divided by 1
    q = kenc.quantize_weight_rtn(torch.from_numpy(w).to(dev), group_size=group, code_bits=code_bits)
    codes, scales = oenc.quantize_weight_rtn(w, group_size=group, code_bits=code_bits)
    np.testing.assert_array_equal(q.scales.cpu().numpy(), scales)
    np.testing.assert_array_equal(_u(q.codes), codes)
    assert q.code_bits == code_bits and q.group_size == group
    p = kenc.quantize_weight_rtn(w, group_size=group, code_bits=code_bits, scale_estimator="percentile_99")
    ref = (np.percentile(np.abs(w.reshape(96, -1, group)), 99.0, axis=2).astype(np.float32)
           / np.float32(np.abs(oenc.grid(code_bits)).max()))
    np.testing.assert_allclose(p.scales.float().cpu().numpy(), ref.astype(np.float16).astype(np.float32),
                               rtol=2 ** -10)


def test_quantized_vq_linear_from_weights(dev):
    rng = np.random.default_rng(11)
    K, N = 512, 64
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    signs = np.where(rng.integers(0, 2, K) == 1, 1.0, -1.0).astype(np.float32)
    layer = keep_amd.QuantizedVQLinear.from_weights(torch.from_numpy(w).to(dev), group_size=256, code_bits=16,
                                                    rht_signs=torch.from_numpy(signs).to(dev))
    codes, scales = oenc.quantize_weight_rtn(orht.apply_rht_f32(w, signs), group_size=256, code_bits=16)
    np.testing.assert_array_equal(_u(layer.codes), codes)
    np.testing.assert_array_equal(layer.scales.cpu().numpy(), scales)
    x = torch.from_numpy(rng.standard_normal((3, K)).astype(np.float32)).to(dev)
    y = layer(x).cpu().numpy().astype(np.float64)
    deq = e8p.decode_weight_matrix(codes, scales.astype(np.float32), code_bits=16, dtype=np.float64)
    want = orht.apply_rht(x.cpu().numpy(), signs) @ deq.T
    assert np.abs(y - want).max() <= 2e-3 * np.abs(want).max()


@pytest.mark.parametrize("code_bits,transform", [(8, None), (16, None), (16, "rht"), (8, "rotation")])
def test_quantized_vq_switch_linear_from_weights(dev, code_bits, transform):
    """Stacked experts ``[E, out, in]`` (switch_linear.py:527-571), with an
    all-zero row and an all-zero group: codes and fp16 scales bit for bit
    against the oracle RTN run per expert on the same transformed weights,
    then a routed forward against the float64 dequantised product."""
    print(f"switch from_weights: code_bits={code_bits} transform={transform}", flush=True)
    rng = np.random.default_rng(21 + code_bits)
    E, N, K, g = 5, 48, 512, 128
    w = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    w[1, 3] = 0.0
    w[2, 5, :g] = 0.0
    kw, xform = {}, (lambda a: a)
    if transform == "rht":
        signs = np.where(rng.integers(0, 2, K) == 1, 1.0, -1.0).astype(np.float32)
        kw["rht_signs"] = torch.from_numpy(signs).to(dev)
        wt = orht.apply_rht_f32(w, signs)  # the GPU RHT is this float32 transform, bit for bit
        xform = lambda a: orht.apply_rht(a, signs)  # noqa: E731
    elif transform == "rotation":
        rot = np.linalg.qr(rng.standard_normal((K, K)))[0].astype(np.float32)
        kw["rotation_matrix"] = torch.from_numpy(rot).to(dev)
        # the product's rounding is the GPU GEMM's: take it from there, and pin it to float64 separately
        wt = (torch.from_numpy(w).to(dev) @ torch.from_numpy(rot).to(dev)).cpu().numpy()
        assert np.abs(wt - w.astype(np.float64) @ rot.astype(np.float64)).max() <= 1e-5
        xform = lambda a: a @ rot.astype(np.float64)  # noqa: E731
    else:
        wt = w
    layer = keep_amd.QuantizedVQSwitchLinear.from_weights(torch.from_numpy(w).to(dev), group_size=g,
                                                          code_bits=code_bits, **kw)
    assert tuple(layer.codes.shape) == (E, N, K // 8) and tuple(layer.scales.shape) == (E, N, K // g)
    ref = [oenc.quantize_weight_rtn(wt[e], group_size=g, code_bits=code_bits) for e in range(E)]
    for e, (codes, scales) in enumerate(ref):
        np.testing.assert_array_equal(_u(layer.codes[e]), codes, err_msg=f"expert {e}")
        np.testing.assert_array_equal(layer.scales[e].cpu().numpy(), scales, err_msg=f"expert {e}")
    assert (ref[1][1][3] == 0).all()  # the zero row stays zero under any transform
    assert transform is not None or ref[2][1][5, 0] == 0  # the zero group only untransformed (RHT mixes a row)
    T, k = 4, 3
    x = rng.standard_normal((T, K)).astype(np.float32)
    idx = rng.integers(0, E, (T, k)).astype(np.int32)
    y = layer(torch.from_numpy(x).to(dev), torch.from_numpy(idx).to(dev)).cpu().numpy().astype(np.float64)
    deq = [e8p.decode_weight_matrix(c, s.astype(np.float32), code_bits=code_bits, dtype=np.float64) for c, s in ref]
    xt = xform(x.astype(np.float64))
    want = np.stack([np.stack([deq[idx[t, j]] @ xt[t] for j in range(k)]) for t in range(T)])
    assert y.shape == want.shape
    assert np.abs(y - want).max() <= 2e-3 * np.abs(want).max()
    with pytest.raises(ValueError, match="3D"):
        keep_amd.QuantizedVQSwitchLinear.from_weights(torch.from_numpy(w[0]).to(dev), group_size=g)
