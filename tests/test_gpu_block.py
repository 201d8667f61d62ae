"""GPU parity of the steps either side of the routed experts against
oracle/block.py:

- keep_rmsnorm_quant_rht, in three parts: (a) the RMSNorm output within one
  ulp of the row dtype of the oracle's (the fp32 sum of squares runs in
  another order); (b) the FP8 act-quant of the GPU's own normed rows equal to
  the oracle's bit for bit; (c) with signs, the RHT of those values equal to
  the float32 RHT restatement bit for bit;
- keep_moe_combine_add bit for bit (fp32 sums in the reference's order);
- RoutedVQMoE with a shared expert and the residual add, decode (T = 1, the
  fused layer), few tokens and prefill, within 2e-3 of the C oracle plus the
  rounding of the bf16 output.
"""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import block as kblock
from keep_amd import synth
from oracle import block, cpu, e8p, ops
from oracle import rht as orht

pytestmark = pytest.mark.gpu
NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}
ULP = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


@pytest.mark.parametrize("n,T,xdt,blk,pow2", [(4096, 1, torch.bfloat16, 128, True),
                                             (4096, 7, torch.bfloat16, 128, False),
                                             (8192, 3, torch.float16, 128, True), (64, 5, torch.float32, 16, False),
                                             (512, 2, torch.bfloat16, 512, True), (2048, 4, torch.float16, 0, False)])
def test_rmsnorm_quant_rht_vs_oracle(dev, n, T, xdt, blk, pow2):
    print(f"rmsnorm_quant_rht: n={n} T={T} x={xdt} block={blk} pow2={pow2}", flush=True)
    rng = np.random.default_rng(n + T)
    x = torch.from_numpy((rng.standard_normal((T, n)) * 3).astype(np.float32)).to(xdt).to(dev)
    gamma = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(xdt).to(dev)
    signs = torch.from_numpy(np.where(rng.integers(0, 2, n) == 1, 1.0, -1.0).astype(np.float32)).to(dev)
    eps = 1e-6
    q, y = kblock.rmsnorm_quant_rht(x, gamma, eps, quant_block=blk, pow2_scales=pow2, return_normed=True)
    name = NAMES[xdt]
    xf, gf = x.float().cpu().numpy(), gamma.float().cpu().numpy()
    # (a) the normed rows
    y_o = block.rmsnorm(xf, gf, eps, name)
    y_g = y.float().cpu().numpy()
    assert (np.abs(y_g - y_o) <= ULP[xdt] * np.abs(y_o) + 1e-30).all(), "normed rows beyond one ulp"
    # (b) the act-quant of the GPU's normed rows, bit for bit
    q_o = block.act_quant(y_g, blk, pow2, name) if blk else y_g
    np.testing.assert_array_equal(q.float().cpu().numpy(), q_o)
    # (c) the RHT of those values (float32 butterflies in the reference's stage order)
    r = kblock.rmsnorm_quant_rht(x, gamma, eps, quant_block=blk, pow2_scales=pow2, rht_signs=signs,
                                 out_dtype=torch.float32)
    np.testing.assert_array_equal(r.cpu().numpy(), orht.apply_rht_f32(q_o, signs.cpu().numpy()))
    np.testing.assert_allclose(r.cpu().numpy(), orht.apply_rht(q_o, signs.cpu().numpy()), rtol=0, atol=1e-4 * 3)


def test_rmsnorm_quant_rht_rejects(dev):
    with pytest.raises(ValueError, match="power of two"):
        kblock.rmsnorm_quant_rht(torch.zeros((2, 96), device=dev))
    with pytest.raises(ValueError, match="quant_block"):
        kblock.rmsnorm_quant_rht(torch.zeros((2, 128), device=dev), quant_block=256)


@pytest.mark.parametrize("sdt,rdt,odt", [(torch.float32, torch.bfloat16, torch.bfloat16),
                                         (torch.bfloat16, None, torch.float32), (None, torch.float16, torch.float16),
                                         (None, None, torch.bfloat16)])
def test_combine_add_bit_exact(dev, sdt, rdt, odt):
    rng = np.random.default_rng(3)
    n = 4096 * 3 + 5  # a ragged tail
    routed = torch.from_numpy((rng.standard_normal(n) * 100).astype(np.float32)).to(dev)
    sh = None if sdt is None else torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(sdt).to(dev)
    res = None if rdt is None else torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(rdt).to(dev)
    out = kblock.combine_add(routed, sh, res, odt)
    want = block.shared_combine(routed.cpu().numpy(), None if sh is None else sh.float().cpu().numpy(),
                                None if res is None else res.float().cpu().numpy(), NAMES[odt])
    np.testing.assert_array_equal(out.float().cpu().numpy(), want)


def _glu(dev, E, H, I, seeds, limit):
    ps = (synth.projection(E, I, H, seed=seeds[0], device=dev), synth.projection(E, I, H, seed=seeds[1], device=dev),
          synth.projection(E, H, I, seed=seeds[2], device=dev))

    def lin(p, K, N):
        return keep_amd.QuantizedVQSwitchLinear(input_dims=K, output_dims=N, num_experts=E, codes=p.codes,
                                                scales=p.scales, group_size=K, code_bits=16)

    glu = keep_amd.QuantizedVQSwitchGLU(gate_proj=lin(ps[0], H, I), up_proj=lin(ps[1], H, I),
                                        down_proj=lin(ps[2], I, H), activation=keep_amd.LimitedSwiGLU(limit))
    return glu, ps


def _host(p):
    return p.codes.cpu().numpy().view(np.uint16), p.scales.float().cpu().numpy()


@pytest.mark.parametrize("T", [1, 4, 160])
def test_routed_moe_with_shared_expert_and_residual(dev, T):
    """config 2's routed layer plus a 2048-wide shared expert and the residual
    stream (bf16 output): routed and shared sums from the C oracle (each with h
    in bf16, the shared expert as a one-expert MoE of weight 1), added by the
    oracle's combine."""
    E, H, I, k, limit = 384, 4096, 2048, 6, 10.0
    print(f"routed + shared + residual: T={T}", flush=True)
    glu, (gate, up, down) = _glu(dev, E, H, I, (1, 2, 3), limit)
    shared, (sg, su, sd) = _glu(dev, 1, H, I, (7, 8, 9), limit)
    moe = keep_amd.RoutedVQMoE(glu, top_k=k, swiglu_limit=limit, shared_experts=shared, out_dtype=torch.bfloat16)
    x = synth.rht_activations(T, H, seed=T, device=dev, dtype=torch.bfloat16)
    z = synth.router_logits(T, E, seed=T + 1, device=dev)
    h = torch.from_numpy(np.random.default_rng(T).standard_normal((T, H)).astype(np.float32) * 50).to(
        torch.bfloat16).to(dev)
    out, r = moe(x, z, residual=h)
    assert out.dtype == torch.bfloat16 and out.shape == (T, H)
    tab = e8p.e8p_packed_abs_grid()
    xf = x.float().cpu().numpy()
    idx = r.idx.cpu().numpy()
    used = np.unique(idx)
    sel = torch.from_numpy(used).to(dev).long()
    pick = lambda p: (p.codes[sel].cpu().numpy().view(np.uint16), p.scales[sel].float().cpu().numpy())  # noqa: E731
    local = np.searchsorted(used, idx).astype(np.int32)
    routed = cpu.moe_decode(xf, local, r.weight.cpu().numpy(), pick(gate), pick(up), pick(down), tab, limit=limit)
    sh = cpu.moe_decode(xf, np.zeros((T, 1), np.int32), np.ones((T, 1), np.float32), _host(sg), _host(su),
                        _host(sd), tab, limit=limit)
    want = block.shared_combine(routed, sh, h.float().cpu().numpy(), "float32").astype(np.float64)
    g = out.float().cpu().numpy()
    err = ops.max_rel_err(g, want)
    assert err <= 2e-3 + 2.0 ** -9, f"max rel err {err:.3e}"
    # the parts on their own: the module's routed output and shared output
    routed_g, _ = keep_amd.RoutedVQMoE(glu, top_k=k, swiglu_limit=limit)(x, z)
    assert ops.max_rel_err(routed_g.cpu().numpy(), routed) <= 2e-3
    assert ops.max_rel_err(moe.shared(x).cpu().numpy(), sh) <= 2e-3
    np.testing.assert_array_equal(
        g, block.shared_combine(routed_g.cpu().numpy(), moe.shared(x).cpu().numpy(), h.float().cpu().numpy(),
                                "bfloat16"))
