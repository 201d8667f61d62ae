"""GPU parity of the activation RHT (``keep_rht``) against the float32 oracle.

The kernel runs the reference's float32 butterflies in the reference's stage
order (``src/keep/quant/rht.py:34-66``), so float32 outputs are compared bit
for bit with ``oracle.rht.hadamard_f32``; fp16 / bf16 outputs are that float32
result rounded to nearest even, also bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import rht as orht

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda", 0)


def _ref(x32, s, mode):
    if mode == "fwd":
        return orht.apply_rht_f32(x32, s)
    if mode == "inv":
        return orht.apply_inverse_rht_f32(x32, s)
    return orht.hadamard_f32(x32)


@pytest.mark.parametrize("n", [16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192])
@pytest.mark.parametrize("mode", ["fwd", "inv", "plain"])
def test_rht_f32_bit_exact(dev, n, mode):
    from keep_amd import rht

    print(f"keep_rht f32 n={n} mode={mode}", flush=True)
    rng = np.random.default_rng(n + len(mode))
    for T in (1, 3, 37):
        x = rng.standard_normal((T, n)).astype(np.float32) * 3
        s = orht.deterministic_rht_signs(n, seed=n).astype(np.float32)
        xd = torch.from_numpy(x).to(dev)
        if mode == "fwd":
            y = rht.apply_rht(xd, torch.from_numpy(s))
        elif mode == "inv":
            y = rht.apply_inverse_rht(xd, torch.from_numpy(s))
        else:
            y = rht.fwht(xd)
        want = _ref(x, s, mode)
        got = y.cpu().numpy()
        assert got.dtype == np.float32
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
def test_rht_dtypes_round_from_f32(dev, xdt, odt):
    from keep_amd import rht

    print(f"keep_rht dtypes x={xdt} out={odt}", flush=True)
    n, T = 4096, 5
    rng = np.random.default_rng(3)
    xt = torch.from_numpy(rng.standard_normal((T, n)).astype(np.float32)).to(xdt)
    s = orht.deterministic_rht_signs(n, seed="layer.0").astype(np.float32)
    y = rht.apply_rht(xt.to(dev), torch.from_numpy(s), out_dtype=odt)
    assert y.dtype == odt and y.shape == (T, n)
    want = torch.from_numpy(orht.apply_rht_f32(xt.float().numpy(), s)).to(odt)
    assert torch.equal(y.cpu().view(torch.int16) if odt != torch.float32 else y.cpu().view(torch.int32),
                       want.view(torch.int16) if odt != torch.float32 else want.view(torch.int32))
    # round trip (float32 path): inverse(forward(x)) == x to float32 rounding
    x32 = xt.float().to(dev)
    back = rht.apply_inverse_rht(rht.apply_rht(x32, torch.from_numpy(s)), torch.from_numpy(s))
    torch.testing.assert_close(back, x32, rtol=0, atol=2e-5)


def test_rht_edges_and_errors(dev):
    from keep_amd import rht

    print("keep_rht edges", flush=True)
    empty = rht.apply_rht(torch.empty((0, 64), device=dev), torch.ones(64))
    assert empty.shape == (0, 64)
    x3 = torch.randn(2, 3, 256, device=dev)
    y3 = rht.fwht(x3)
    want = orht.hadamard_f32(x3.cpu().numpy())
    np.testing.assert_array_equal(y3.cpu().numpy().view(np.uint32), want.view(np.uint32))
    for n in (8, 12, 16384):
        with pytest.raises(ValueError):
            rht.fwht(torch.zeros(1, n, device=dev))
    with pytest.raises(ValueError):
        rht.apply_rht(torch.zeros(1, 64, device=dev), torch.ones(32))
    bad = torch.ones(64)
    bad[5] = 0.5  # signs must be -1 or 1, as _validate_signs_np requires
    with pytest.raises(ValueError, match="-1 or 1"):
        rht.apply_rht(torch.zeros(1, 64, device=dev), bad)
    with pytest.raises(ValueError, match="-1 or 1"):
        rht.apply_inverse_rht(torch.zeros(1, 64, device=dev), bad.to(dev))
