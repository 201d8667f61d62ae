"""GPU parity of the residual tier alone (keep_e8_1bit_matvec behind
e8_1bit_m1_token_layout / e8_1bit_m1_per_route) against a float64 dense
decode, with the reference's cases (tests/test_e8_1bit_m1.py:39-70): group
sizes 32 / 64 / 256, a ragged last row tile, routes at NO_RESIDUAL writing
zeros, fp32 / bf16 / fp16 activations."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import ops as kops
from oracle import e8p, ops

pytestmark = pytest.mark.gpu
NONE = kops.NO_RESIDUAL


def _layer(E, N, K, group_size, seed, dev):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, (E, N, K // 8), dtype=np.uint8)
    scales = rng.uniform(0.01, 0.2, (E, N, K // group_size)).astype(np.float16)
    dense = e8p.decode_e8_1bit(codes).astype(np.float64).reshape(E, N, K)
    dense *= np.repeat(scales.astype(np.float64), group_size, axis=-1)
    return torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev), dense


@pytest.mark.parametrize("group_size,K,N", [(32, 128, 96), (64, 768, 93), (256, 4096, 64)])
@pytest.mark.parametrize("xdt,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2), (torch.float16, 2e-3)])
def test_both_layouts_match_the_dense_decode(dev, group_size, K, N, xdt, tol):
    codes, scales, dense = _layer(6, N, K, group_size, seed=3, dev=dev)
    book = torch.from_numpy(kops.pair_packed(e8p.e8_1bit_packed()).view(np.int32)).to(dev)
    rng = np.random.default_rng(4)
    rhs = np.array([[5, 0, 3], [NONE, 2, 2], [1, NONE, 4]], dtype=np.uint32)

    def rows(n):
        x = torch.from_numpy(rng.normal(size=(n, K)).astype(np.float32)).to(dev).to(xdt)
        return x, x.float().cpu().numpy().astype(np.float64)

    def ref(x_row, e):
        return np.zeros(N) if e == NONE else x_row @ dense[e].T

    def close(got, want):
        assert got.dtype == (xdt if xdt != torch.float32 else torch.float32)
        g = got.float().cpu().numpy().astype(np.float64)
        assert g.shape == want.shape
        assert ops.max_rel_err(g, want) <= tol

    x, xn = rows(3)
    got = keep_amd.e8_1bit_m1_token_layout(x, codes, scales, book, torch.from_numpy(rhs.view(np.int32)).to(dev),
                                           output_dims=N)
    want = np.stack([[ref(xn[t], e) for e in rhs[t]] for t in range(3)])
    close(got, want)
    assert (got[1, 0] == 0).all() and (got[2, 1] == 0).all()
    x, xn = rows(9)
    got = keep_amd.e8_1bit_m1_per_route(x, codes, scales, book, rhs.reshape(-1), output_dims=N)
    close(got, np.stack([ref(xn[r], e) for r, e in enumerate(rhs.reshape(-1))]))


def test_out_of_range_index_other_than_none_is_nan(dev):
    codes, scales, _ = _layer(4, 64, 256, 256, seed=5, dev=dev)
    x = torch.randn(2, 256, device=dev)
    got = keep_amd.e8_1bit_m1_per_route(x, codes, scales, None, np.array([9, NONE], dtype=np.uint32), output_dims=64)
    assert torch.isnan(got[0]).all() and (got[1] == 0).all()
