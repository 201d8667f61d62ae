"""GPU parity: dual top-k router (exact indices), device route plan (exact),
MFMA grouped GEMM, verify rows and the fused MoE decode layer."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import synth
from oracle import cpu, e8p, ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
TOL_BF16_OUT = TOL + 2.0 ** -9  # a bf16-stored output adds at most 2**-9 relative rounding


def _t(a, dev):
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check(got, want, tol=TOL):
    g = got.float().cpu().numpy()
    err = ops.max_rel_err(g, want)
    assert err <= tol, f"max rel err {err:.3e}"
    assert ops.elementwise_ok(g, want, rtol=tol), "elementwise bound violated"
    return err


@pytest.mark.parametrize("T,E,k,func", [(1, 384, 6, "softmax"), (64, 384, 6, "softmax"), (33, 288, 8, "sigmoid"),
                                        (17, 256, 8, "sqrtsoftplus"), (5, 1024, 32, "softmax")])
def test_router_indices_exact_unmasked(dev, T, E, k, func):
    z = synth.router_logits(T, E, seed=T + E, device=dev)
    r = keep_amd.router_dual_topk(z, k, score_func=func, route_scale=2.5)
    idx, w, want, ws, admit = ops.router_dual_topk(z.cpu().numpy(), np.zeros(E), np.zeros(E), k, func=func,
                                                   route_scale=2.5)
    np.testing.assert_array_equal(r.idx.cpu().numpy(), idx)
    np.testing.assert_array_equal(r.want.cpu().numpy(), want)
    np.testing.assert_allclose(r.weight.cpu().numpy(), w, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(r.want_score.cpu().numpy(), ws, rtol=2e-6, atol=1e-9)


@pytest.mark.parametrize("T", [1, 512])
def test_router_residency_config5(dev, T):
    E, k, tau = 288, 8, 0.3
    z = synth.router_logits(T, E, seed=7, device=dev)
    mask = synth.resident_mask(E, frac=0.5, seed=8)
    bias = keep_amd.resident_bias(torch.from_numpy(mask).to(dev))
    r = keep_amd.router_dual_topk(z, k, bias_served=bias, tau=tau)
    idx, w, want, ws, admit = ops.router_dual_topk(z.cpu().numpy(), bias.cpu().numpy(), np.zeros(E), k, tau=tau)
    np.testing.assert_array_equal(r.idx.cpu().numpy(), idx)
    np.testing.assert_array_equal(r.want.cpu().numpy(), want)
    np.testing.assert_array_equal(r.admit.cpu().numpy().astype(bool), admit)
    assert mask[r.idx.cpu().numpy()].all()  # served is always resident here (144 > k)
    np.testing.assert_allclose(r.weight.cpu().numpy().sum(-1), 1.0, rtol=1e-5)


def test_router_fewer_resident_than_k(dev):
    E, k = 64, 6
    z = synth.router_logits(9, E, seed=3, device=dev)
    bias = torch.full((E,), float("-inf"), device=dev)
    bias[[5, 40]] = 0.0
    r = keep_amd.router_dual_topk(z, k, bias_served=bias)
    idx, w, *_ = ops.router_dual_topk(z.cpu().numpy(), bias.cpu().numpy(), np.zeros(E), k)
    np.testing.assert_array_equal(r.idx.cpu().numpy(), idx)
    wg = r.weight.cpu().numpy()
    assert ((wg > 0).sum(-1) == 2).all()
    np.testing.assert_allclose(wg, w, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("R,E,tile,skew,bad", [(6, 384, 64, False, 0), (384, 384, 4, False, 0),
                                                (12288, 384, 64, False, 0), (1000, 7, 16, False, 0),
                                                (0, 5, 8, False, 0), (16384, 384, 64, False, 0),
                                                (20000, 384, 64, False, 0), (5000, 1024, 32, False, 0),
                                                (1025, 1, 4, False, 0), (12288, 384, 64, True, 0),
                                                (300, 16, 8, False, 21), (20000, 384, 64, False, 130),
                                                (48, 384, 4, False, 0), (96, 384, 4, True, 0),
                                                (128, 16, 4, False, 9), (127, 1024, 3, True, 5),
                                                (64, 1, 4, False, 0), (65, 2, 64, False, 3), (1, 384, 4, False, 0),
                                                (100, 7, 3, True, 100), (128, 384, 128, False, 0)])
def test_route_plan_exact(dev, R, E, tile, skew, bad):
    # up to 128 routes one wave ranks them all (two per lane, across both halves); beyond, each of the
    # plan's 16 waves ranks a contiguous range of max(64, ceil(R / 16)) routes; `bad` routes get expert
    # ids outside [0, E): they sort last, in tiles of expert -1
    rng = np.random.default_rng(R + E)
    rhs = rng.integers(0, E, size=R).astype(np.int32)
    if skew:  # a few hot experts: long same-expert runs inside each wave
        rhs = ((rng.zipf(1.3, size=R) - 1) % E).astype(np.int32)
    if bad:
        at = rng.choice(R, bad, replace=False)
        rhs[at] = rng.choice(np.array([-1, -7, E, E + 3], dtype=np.int32), bad)
    order, inv, counts, offsets, te, to, tc, nt = keep_amd.route_plan(_t(rhs, dev), E, tile)
    o_order, o_inv, o_counts, o_offsets, o_te, o_to, o_tc = ops.route_plan(rhs, E, tile)
    np.testing.assert_array_equal(order.cpu().numpy(), o_order)
    np.testing.assert_array_equal(inv.cpu().numpy(), o_inv)
    np.testing.assert_array_equal(counts.cpu().numpy(), o_counts)
    np.testing.assert_array_equal(offsets.cpu().numpy(), o_offsets)
    n = len(o_te)
    assert int(nt.item()) == int((o_te >= 0).sum())  # valid tiles only
    np.testing.assert_array_equal(te.cpu().numpy()[:n], o_te)
    np.testing.assert_array_equal(to.cpu().numpy()[:n], o_to)
    np.testing.assert_array_equal(tc.cpu().numpy()[:n], o_tc)
    assert (tc.cpu().numpy()[n:] == 0).all()
    assert int((o_te < 0).sum()) == -(-bad // tile)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 4])
def test_grouped_gemm_sorted_routes(dev, xdt, G):
    E, N, K, T, k = 12, 320, 512, 70, 4
    codes, scales = synth.projection_np(E, N, K, group_size=K // G, seed=G)
    rhs = synth.zipf_routes(T, E, k, seed=3)
    x = synth.rht_activations(T, K, seed=4, device=dev, dtype=xdt)
    with keep_amd.trace_gather_vqmm_calls() as tr:
        y = keep_amd.gather_vqmm(x, _t(codes, dev), _t(scales, dev), None, _t(rhs, dev), input_dims=K,
                                 output_dims=N, group_size=K // G, code_bits=16, route_strategy="sorted_tiled")
    assert tr[0]["implementation"] == "mfma_grouped_gemm"
    want = ops.gather_token(x.float().cpu().numpy(), codes, scales, rhs)
    _check(y, want, TOL_BF16_OUT if xdt == torch.bfloat16 else TOL)
    # fp32 output of the same GEMM holds 2e-3
    flat = _t(rhs.reshape(-1), dev)
    order, inverse, _, _, te, to, tc, _ = keep_amd.route_plan(flat, E, 64)
    lhs = (torch.arange(flat.numel(), device=dev, dtype=torch.int32) // k)[order.long()].contiguous()
    y32 = keep_amd.ops.grouped_gemm(x, _t(codes, dev), _t(scales, dev), keep_amd.ops._default_codebook(16, dev),
                                    (te, to, tc), lhs=lhs, routes=flat.numel(), input_dims=K, output_dims=N,
                                    group_size=K // G, out_dtype=torch.float32)
    _check(y32[inverse.long()].reshape(T, k, N), want)


def test_sorted_routes_entry_with_presorted_x(dev):
    E, N, K, R = 5, 256, 256, 150
    codes, scales = synth.projection_np(E, N, K, seed=9)
    rng = np.random.default_rng(10)
    rhs = np.sort(rng.integers(0, E, size=R)).astype(np.int32)
    x = torch.from_numpy(rng.standard_normal((R, K)).astype(np.float16)).to(dev)
    lhs = np.arange(R, dtype=np.int32)
    y = keep_amd.gather_vqmm_sorted_routes(x, _t(codes, dev), _t(scales, dev), None, _t(rhs, dev), _t(lhs, dev),
                                           input_dims=K, output_dims=N, group_size=K, code_bits=16,
                                           x_pre_sorted=True, validate_indices=True)
    _check(y, ops.gather_routes(x.float().cpu().numpy(), codes, scales, rhs, lhs))


@pytest.mark.parametrize("M", [8, 16, 64])
def test_verify_rows_expert_grouping_bit_identical_to_flat(dev, M):
    E, N, K, k = 384, 64, 4096, 6
    codes = torch.randint(-32768, 32768, (E, N, K // 8), dtype=torch.int16, device=dev)
    scales = torch.exp(torch.randn((E, N, 1), device=dev) * 0.3).half()
    x = synth.rht_activations(M, K, seed=M, device=dev)
    z = synth.router_logits(M, E, seed=M + 1, device=dev)
    rhs = keep_amd.router_dual_topk(z, k).idx
    flat = keep_amd.gather_vqmm_verify_rows(x, codes, scales, None, rhs, input_dims=K, output_dims=N,
                                            group_size=K, grouping="flat")
    grouped = keep_amd.gather_vqmm_verify_rows(x, codes, scales, None, rhs, input_dims=K, output_dims=N,
                                               group_size=K, grouping="expert", m_rows=4)
    assert torch.equal(flat, grouped)
    r = rhs.cpu().numpy()
    used = np.unique(r)
    c_np = codes.cpu().numpy().view(np.uint16)
    s_np = scales.cpu().numpy()
    want = np.zeros((M, k, N))
    for e in used:
        W = ops.dense(c_np[e], s_np[e])
        for t, j in zip(*np.nonzero(r == e)):
            want[t, j] = W @ x[t].float().cpu().numpy()
    _check(flat, want)


def _verify_routes(pattern, M, k, E, rng):
    """Verify-row routing patterns of increasing same-expert overlap (as the
    reference's tests/test_gather_vqmm_verify_rows.py:_routes)."""
    if pattern == "uniform":
        return rng.integers(0, E, size=(M, k), dtype=np.int32)
    if pattern == "skewed":
        return rng.integers(0, max(2, E // 3), size=(M, k), dtype=np.int32)
    if pattern == "duplicate":
        return np.tile(rng.choice(E, size=k, replace=False).astype(np.int32), (M, 1))
    return np.zeros((M, k), dtype=np.int32)  # single expert: full tiles, then a partial tail


@pytest.mark.parametrize("M,pattern,xdt", [(2, "uniform", torch.float16), (8, "skewed", torch.bfloat16),
                                           (8, "duplicate", torch.float32), (33, "single_expert", torch.float16),
                                           (64, "uniform", torch.bfloat16)])
def test_verify_rows_uint8_codes(dev, M, pattern, xdt):
    """The reference verify operator's own format: uint8 codes indexing the
    packed 8-bit E8 table (gather_vqmm.py:387-388). Expert grouping is bit
    identical to flat and to the M = 1 gather run per verify row; both match the
    dense 8-bit decode (oracle) within 2e-3. N = 93 leaves a ragged row block."""
    E, N, K, k, G = 8, 93, 1024, 6, 512
    rng = np.random.default_rng(M)
    codes = torch.from_numpy(rng.integers(0, 256, size=(E, N, K // 8), dtype=np.uint8)).to(dev)
    scales = torch.from_numpy(np.exp(rng.normal(0, 0.3, size=(E, N, K // G))).astype(np.float16)).to(dev)
    x = synth.rht_activations(M, K, seed=M + 7, device=dev).to(xdt)
    rhs = torch.from_numpy(_verify_routes(pattern, M, k, E, rng)).to(dev)
    flat = keep_amd.gather_vqmm_verify_rows(x, codes, scales, None, rhs, input_dims=K, output_dims=N,
                                            group_size=G, grouping="flat")
    for mr in (1, 4, 8):
        grouped = keep_amd.gather_vqmm_verify_rows(x, codes, scales, None, rhs, input_dims=K, output_dims=N,
                                                   group_size=G, grouping="expert", m_rows=mr)
        assert torch.equal(flat, grouped), f"expert grouping (m_rows={mr}) differs from flat"
    for t in range(M):
        one = keep_amd.gather_vqmm(x[t:t + 1], codes, scales, None, rhs[t:t + 1], input_dims=K, output_dims=N,
                                   group_size=G, code_bits=8)
        assert torch.equal(one[0], flat[t]), f"verify row {t} differs from the M = 1 gather"
    r = rhs.cpu().numpy()
    c_np, s_np = codes.cpu().numpy(), scales.float().cpu().numpy()
    xf = x.float().cpu().numpy().astype(np.float64)
    want = np.zeros((M, k, N))
    for e in np.unique(r):
        W = ops.dense(c_np[e], s_np[e], code_bits=8)
        for t, j in zip(*np.nonzero(r == e)):
            want[t, j] = W @ xf[t]
    assert flat.dtype == xdt  # the output takes x's dtype, as the reference kernel's OUT_T
    _check(flat, want, {torch.bfloat16: TOL_BF16_OUT, torch.float16: TOL + 2.0 ** -11}.get(xdt, TOL))


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_moe_decode_small_vs_oracle(dev, xdt):
    E, H, I, k, T = 16, 512, 256, 4, 3
    gate = synth.projection_np(E, I, H, group_size=256, seed=1)
    up = synth.projection_np(E, I, H, group_size=256, seed=2)
    down = synth.projection_np(E, H, I, seed=3)
    x = synth.rht_activations(T, H, seed=4, device=dev, dtype=xdt)
    z = synth.router_logits(T, E, seed=5, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    tt = lambda p: (_t(p[0], dev), _t(p[1], dev))  # noqa: E731
    out = keep_amd.moe_decode(x, r.idx, r.weight, tt(gate), tt(up), tt(down), limit=10.0)
    assert out.dtype == torch.float32
    want = ops.moe_layer(x.float().cpu().numpy(), r.idx.cpu().numpy(), r.weight.cpu().numpy(), gate, up, down,
                         limit=10.0, h_round="bfloat16")
    _check(out, want)


def test_moe_layer_config2_full_shape_vs_c_oracle(dev):
    """Config 2 at its real shape: 384 experts, 4096/2048, top-6, batch 1."""
    E, H, I, k = 384, 4096, 2048, 6
    gate = synth.projection(E, I, H, seed=1, device=dev)
    up = synth.projection(E, I, H, seed=2, device=dev)
    down = synth.projection(E, H, I, seed=3, device=dev)
    x = synth.rht_activations(1, H, seed=4, device=dev)
    z = synth.router_logits(1, E, seed=5, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    out = keep_amd.moe_decode(x, r.idx, r.weight, (gate.codes, gate.scales), (up.codes, up.scales),
                              (down.codes, down.scales))
    idx = r.idx.cpu().numpy()
    used = np.unique(idx)
    sub = {e: i for i, e in enumerate(used)}
    pick = lambda p: (p.codes[torch.from_numpy(used).to(dev).long()].cpu().numpy().view(np.uint16),  # noqa: E731
                      p.scales[torch.from_numpy(used).to(dev).long()].float().cpu().numpy())
    g, u, d = pick(gate), pick(up), pick(down)
    local = np.vectorize(sub.get)(idx).astype(np.int32)
    want = cpu.moe_decode(x.float().cpu().numpy(), local, r.weight.cpu().numpy(), g, u, d, e8p.e8p_packed_abs_grid())
    _check(out, want)
    zi, zw, *_ = ops.router_dual_topk(z.cpu().numpy(), np.zeros(E), np.zeros(E), k)
    np.testing.assert_array_equal(idx, zi)


def test_routed_moe_module_prefill_matches_decode_path(dev):
    E, H, I, k, T = 32, 512, 256, 6, 48  # 288 routes -> MFMA prefill path
    gate = synth.projection_np(E, I, H, seed=11)
    up = synth.projection_np(E, I, H, seed=12)
    down = synth.projection_np(E, H, I, seed=13)
    mk = lambda p, i, o: keep_amd.QuantizedVQSwitchLinear(input_dims=i, output_dims=o, num_experts=E,  # noqa: E731
                                                          codes=_t(p[0], dev), scales=_t(p[1], dev), group_size=i,
                                                          code_bits=16)
    glu = keep_amd.QuantizedVQSwitchGLU(gate_proj=mk(gate, H, I), up_proj=mk(up, H, I), down_proj=mk(down, I, H),
                                        activation=keep_amd.LimitedSwiGLU(10.0, fp32=True))
    x = synth.rht_activations(T, H, seed=14, device=dev)
    z = synth.router_logits(T, E, seed=15, device=dev)
    moe = keep_amd.RoutedVQMoE(glu, top_k=k, swiglu_limit=10.0, decode_max_tokens=0)
    out, r = moe(x, z)
    want = ops.moe_layer(x.float().cpu().numpy(), r.idx.cpu().numpy(), r.weight.cpu().numpy(), gate, up, down,
                         limit=10.0, h_round="bfloat16")
    _check(out, want)
    moe_dec = keep_amd.RoutedVQMoE(glu, top_k=k, swiglu_limit=10.0, decode_max_tokens=64)
    out2, _ = moe_dec(x, z)
    _check(out2, want)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("gh,gi", [(2048, 1024), (512, 256)])
def test_moe_decode_tiles_and_packed_table_paths(dev, xdt, gh, gi):
    """H = 2048, I = 1024, three tokens: the int8 tiles kernels and the packed-table kernels
    (prepared=False) against the oracle."""
    E, H, I, k, T = 32, 2048, 1024, 4, 3
    gate = synth.projection_np(E, I, H, group_size=gh, seed=21)
    up = synth.projection_np(E, I, H, group_size=gh, seed=22)
    down = synth.projection_np(E, H, I, group_size=gi, seed=23)
    x = synth.rht_activations(T, H, seed=24, device=dev, dtype=xdt)
    z = synth.router_logits(T, E, seed=25, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    tt = lambda p: (_t(p[0], dev), _t(p[1], dev))  # noqa: E731
    tiles = keep_amd.moe_decode(x, r.idx, r.weight, tt(gate), tt(up), tt(down), limit=10.0)
    packed = keep_amd.moe_decode(x, r.idx, r.weight, tt(gate), tt(up), tt(down), limit=10.0, prepared=False)
    want = ops.moe_layer(x.float().cpu().numpy(), r.idx.cpu().numpy(), r.weight.cpu().numpy(), gate, up, down,
                         limit=10.0, h_round="bfloat16")
    _check(tiles, want)
    _check(packed, want)


@pytest.mark.parametrize("T", [1, 3])
def test_moe_decode_config5_shapes_with_absent_experts(dev, T):
    """288 experts, top-8, 4096/1536, half the pool absent: weight-0 routes are skipped."""
    E, H, I, k = 288, 4096, 1536, 8
    gate = synth.projection(E, I, H, seed=31, device=dev)
    up = synth.projection(E, I, H, seed=32, device=dev)
    down = synth.projection(E, H, I, seed=33, device=dev)
    x = synth.rht_activations(T, H, seed=34, device=dev)
    z = synth.router_logits(T, E, seed=35, device=dev)
    mask = torch.from_numpy(synth.resident_mask(E, frac=0.5, seed=36)).to(dev)
    r = keep_amd.router_dual_topk(z, k, bias_served=keep_amd.resident_bias(mask), tau=0.3)
    w = r.weight.clone()
    w[:, -1] = 0.0  # one surplus slot with zero weight per token
    out = keep_amd.moe_decode(x, r.idx, w, (gate.codes, gate.scales), (up.codes, up.scales),
                              (down.codes, down.scales))
    idx = r.idx.cpu().numpy()
    used = np.unique(idx)
    sub = {e: i for i, e in enumerate(used)}
    sel = torch.from_numpy(used).to(dev).long()
    pick = lambda p: (p.codes[sel].cpu().numpy().view(np.uint16), p.scales[sel].float().cpu().numpy())  # noqa: E731
    local = np.vectorize(sub.get)(idx).astype(np.int32)
    want = cpu.moe_decode(x.float().cpu().numpy(), local, w.cpu().numpy(), pick(gate), pick(up), pick(down),
                          e8p.e8p_packed_abs_grid())
    _check(out, want)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("gh,gi", [(1024, 512), (256, 256), (512, 128)])
def test_moe_decode_matrix_core_path(dev, xdt, gh, gi):
    """One token through the int8 tiles kernels where they serve the scale groups (gi = 128 is
    not a multiple of 256: the packed-table kernels), against the oracle and prepared=False."""
    E, H, I, k, T = 32, 1024, 512, 5, 1
    gate = synth.projection_np(E, I, H, group_size=gh, seed=41)
    up = synth.projection_np(E, I, H, group_size=gh, seed=42)
    down = synth.projection_np(E, H, I, group_size=gi, seed=43)
    x = synth.rht_activations(T, H, seed=44, device=dev, dtype=xdt)
    z = synth.router_logits(T, E, seed=45, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    w = r.weight.clone()
    w[0, 2] = 0.0  # a zero-weight route contributes nothing
    tt = lambda p: (_t(p[0], dev), _t(p[1], dev))  # noqa: E731
    out = keep_amd.moe_decode(x, r.idx, w, tt(gate), tt(up), tt(down), limit=10.0)
    ref = keep_amd.moe_decode(x, r.idx, w, tt(gate), tt(up), tt(down), limit=10.0, prepared=False)
    want = ops.moe_layer(x.float().cpu().numpy(), r.idx.cpu().numpy(), w.cpu().numpy(), gate, up, down,
                         limit=10.0, h_round="bfloat16")
    _check(out, want)
    _check(ref, want)
    bad = r.idx.clone()
    bad[0, 1] = E + 3  # out-of-range expert with nonzero weight: the token's row is NaN, not a fault
    out_bad = keep_amd.moe_decode(x, bad, w, tt(gate), tt(up), tt(down), limit=10.0)
    assert torch.isnan(out_bad).all()


def _layer_oracle(x, r_idx, w, gate, up, down, limit=0.0):
    """C-oracle MoE output for one token over the experts actually used."""
    idx = r_idx.cpu().numpy()
    used = np.unique(idx)
    sub = {e: i for i, e in enumerate(used)}
    sel = torch.from_numpy(used).to(gate.codes.device).long()
    pick = lambda p: (p.codes[sel].cpu().numpy().view(np.uint16), p.scales[sel].float().cpu().numpy())  # noqa: E731
    local = np.vectorize(sub.get)(idx).astype(np.int32)
    return cpu.moe_decode(x.float().cpu().numpy(), local, w.cpu().numpy(), pick(gate), pick(up), pick(down),
                          e8p.e8p_packed_abs_grid(), limit=limit)


def test_moe_layer_config2(dev):
    """Config 2 through the routed decode layer: router indices exact, output vs the C oracle and the split path,
    and a second call with other logits on the same h_work (the down launch must see the new routing)."""
    E, H, I, k = 384, 4096, 2048, 6
    gate = synth.projection(E, I, H, seed=1, device=dev)
    up = synth.projection(E, I, H, seed=2, device=dev)
    down = synth.projection(E, H, I, seed=3, device=dev)
    assert keep_amd.moe_layer_supported(E, H, I, k, H, I)
    x = synth.rht_activations(1, H, seed=4, device=dev)
    h_work = torch.empty(k * I, dtype=torch.bfloat16, device=dev)
    for seed in (5, 6):
        z = synth.router_logits(1, E, seed=seed, device=dev)
        out, r = keep_amd.moe_layer(x, z, (gate.codes, gate.scales), (up.codes, up.scales),
                                    (down.codes, down.scales), k=k, h_work=h_work)
        zi, zw, *_ = ops.router_dual_topk(z.cpu().numpy(), np.zeros(E), np.zeros(E), k)
        np.testing.assert_array_equal(r.idx.cpu().numpy(), zi)
        np.testing.assert_allclose(r.weight.cpu().numpy(), zw, rtol=1e-5, atol=1e-7)
        _check(out, _layer_oracle(x, r.idx, r.weight, gate, up, down))
        split = keep_amd.moe_decode(x, r.idx, r.weight, (gate.codes, gate.scales), (up.codes, up.scales),
                                    (down.codes, down.scales))
        _check(out, split.double().cpu().numpy())


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_moe_layer_config5_residency(dev, xdt):
    """Config 5 shapes: half the pool absent (served vs demand), tau admission, group scales."""
    E, H, I, k = 288, 4096, 1536, 8
    gate = synth.projection(E, I, H, group_size=1024, seed=31, device=dev)
    up = synth.projection(E, I, H, group_size=1024, seed=32, device=dev)
    down = synth.projection(E, H, I, group_size=512, seed=33, device=dev)
    x = synth.rht_activations(1, H, seed=34, device=dev, dtype=xdt)
    z = synth.router_logits(1, E, seed=35, device=dev)
    mask = synth.resident_mask(E, frac=0.5, seed=36)
    bias = keep_amd.resident_bias(torch.from_numpy(mask).to(dev))
    out, r = keep_amd.moe_layer(x, z, (gate.codes, gate.scales), (up.codes, up.scales), (down.codes, down.scales),
                                k=k, bias_served=bias, tau=0.3)
    ref = keep_amd.router_dual_topk(z, k, bias_served=bias, tau=0.3)
    oi, ow, owant, osc, oadm = ops.router_dual_topk(z.cpu().numpy(), bias.cpu().numpy().astype(np.float64),
                                                    np.zeros(E), k, tau=0.3)
    np.testing.assert_array_equal(r.idx.cpu().numpy(), oi)
    np.testing.assert_array_equal(r.want.cpu().numpy(), owant)
    np.testing.assert_array_equal(r.admit.cpu().numpy(), oadm.astype(np.uint8))
    for a, b in zip(r, ref):
        assert torch.equal(a, b)  # the fused router is the standalone router, bit for bit
    assert set(r.idx.cpu().numpy().ravel()) <= set(np.flatnonzero(mask))
    _check(out, _layer_oracle(x, r.idx, r.weight, gate, up, down))


def test_moe_layer_rejects_unserved_shapes(dev):
    E, H, I, k = 16, 512, 256, 4
    assert not keep_amd.moe_layer_supported(E, H, I, k, H, I)
    gate = synth.projection(E, I, H, seed=1, device=dev)
    down = synth.projection(E, H, I, seed=3, device=dev)
    x = synth.rht_activations(1, H, seed=4, device=dev)
    z = synth.router_logits(1, E, seed=5, device=dev)
    with pytest.raises(ValueError, match="routed decode layer"):
        keep_amd.moe_layer(x, z, (gate.codes, gate.scales), (gate.codes, gate.scales), (down.codes, down.scales),
                           k=k)
